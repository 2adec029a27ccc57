"""Affine quantized matmul on the GPU: bit-exact unpack + dequantization
(identity probe), bitwise parity with the oracle on every launch shape, batch
invariance at the Llama-3-8B MLP shape."""

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, bits, gen, randn, to_np
from oracle import bi_oracle as ora
from sweep import sweep

pytestmark = pytest.mark.gpu

CASES = [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)]


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _qweights(N, K, bits_, gs, dt, seed, scale=0.02):
    g = gen(seed)
    W = torch.randn((N, K), generator=g) * scale
    return _bi().quantize(W, group_size=gs, bits=bits_, dtype=DT[dt])


@pytest.mark.parametrize("bits_,gs", CASES)
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_dequantization_bit_exact(bits_, gs, dt):
    """x = I_K makes row k of the output exactly W[:, k] as dequantized by the
    kernel (one non-zero product per sum), so unpacking, group indexing and the
    fmaf + rounding are compared bit for bit with the closed form."""
    N, K = 96, 512
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 1000 + gs)
    eye = torch.eye(K, dtype=DT[dt])
    got = _bi().batch_invariant_quantized_matmul(eye.cuda(), wq.cuda(), s.cuda(), b.cuda(),
                                                  group_size=gs, bits=bits_)
    want = ora.dequantize(wq.view(torch.int32).numpy().view(np.uint32), to_np(s), to_np(b), gs, bits_, dt)
    np.testing.assert_array_equal(to_np(got), want.T)


@pytest.mark.parametrize("bits_,gs", CASES)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [1, 9, 40])
def test_quantized_matches_oracle(bits_, gs, dt, M):
    N, K = 200, 1024
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=M + bits_ + gs)
    x = randn((M, K), DT[dt], gen(M))
    got = to_np(_bi().batch_invariant_quantized_matmul(x, wq.cuda(), s.cuda(), b.cuda(),
                                                       group_size=gs, bits=bits_))
    W = ora.dequantize(wq.view(torch.int32).numpy().view(np.uint32), to_np(s), to_np(b), gs, bits_, dt)
    assert_bits_equal(got, ora.matmul(to_np(x), W, dt, kmap="blocked"), f"{dt} {bits_}-bit g{gs} M={M}")


@pytest.mark.parametrize("bits_,gs,K", [(4, 64, 8256), (8, 128, 8320)])
def test_quantized_partial_last_group_long_k(bits_, gs, K):
    """33 K groups, the last cut short, at 5..16 rows: the workgroup-fold GEMV
    with four groups of codes requested ahead and the short group computed
    from global memory. Rows equal the oracle and the same rows alone."""
    N = 136
    wq, s, b = _qweights(N, K, bits_, gs, "bf16", seed=K + bits_)
    W = ora.dequantize(wq.view(torch.int32).numpy().view(np.uint32), to_np(s), to_np(b), gs, bits_, "bf16")
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((16, K), torch.bfloat16, gen(K))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    for M in (5, 8, 16):
        got = run(x[:M])
        rows = sorted({0, M - 1})
        assert_bits_equal(to_np(got)[rows], ora.matmul(to_np(x[rows]), W, "bf16", kmap="blocked"), f"K={K} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs,K", [(4, 64, 1088), (4, 32, 1056), (8, 128, 1152), (8, 32, 288)])
@pytest.mark.parametrize("M", [1, 20, 40])
def test_quantized_partial_last_group(bits_, gs, K, M):
    """K not a multiple of 256: the last K group is cut short (zero padding)."""
    N = 136
    wq, s, b = _qweights(N, K, bits_, gs, "bf16", seed=K + M)
    x = randn((M, K), torch.bfloat16, gen(K))
    got = to_np(_bi().batch_invariant_quantized_matmul(x, wq.cuda(), s.cuda(), b.cuda(), group_size=gs, bits=bits_))
    W = ora.dequantize(wq.view(torch.int32).numpy().view(np.uint32), to_np(s), to_np(b), gs, bits_, "bf16")
    assert_bits_equal(got, ora.matmul(to_np(x), W, "bf16", kmap="blocked"), f"K={K} M={M}")
    one = _bi().batch_invariant_quantized_matmul(x[:1], wq.cuda(), s.cuda(), b.cuda(), group_size=gs, bits=bits_)
    assert bits(one) == bits(torch.tensor(got[:1]).to(torch.bfloat16).cuda())


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (8, 32)])
def test_quantized_launch_shapes_agree(bits_, gs):
    """M = 1 and 16 (the streaming GEMV; 8-bit M = 16 one m-tile), 20 and 32
    (two m-tiles), 33 and 100 (LDS tiles, register fold) give the same bits
    for the same rows."""
    N, K = 512, 2048
    wq, s, b = _qweights(N, K, bits_, gs, "bf16", seed=9)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((100, K), torch.bfloat16, gen(3))
    full = _bi().batch_invariant_quantized_matmul(x, wq, s, b, group_size=gs, bits=bits_)
    for M in (1, 16, 20, 32, 33):
        got = _bi().batch_invariant_quantized_matmul(x[:M], wq, s, b, group_size=gs, bits=bits_)
        assert bits(got) == bits(full[:M]), M


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (4, 128), (8, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantized_mid_m_launch_matches_oracle(bits_, gs, dt):
    """4 < M <= 128 with >= 128 blocks of 64 columns takes the mid-M launch
    (A staged per 256-k group in LDS, B straight to registers): rows of every
    M-tile count equal the oracle bit for bit and equal the same
    rows computed alone (M = 1, the GEMV launch), bit for bit."""
    N, K = 8200, 768          # 129 column blocks, the last one partial
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 7 + gs)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((128, K), DT[dt], gen(11))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    W = ora.dequantize(wq.cpu().view(torch.int32).numpy().view(np.uint32), to_np(s.cpu()), to_np(b.cpu()),
                       gs, bits_, dt)
    cols = np.r_[0:40, N - 40:N]
    for M in (5, 17, 33, 64, 100, 128):
        got = run(x[:M])
        rows = sorted({0, M // 2, M - 1})
        want = ora.matmul(to_np(x[rows]), W[cols], dt, kmap="blocked")
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"{dt} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (8, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_quantized_stream_launch_up_to_16_rows(bits_, gs, dt):
    """M <= 16 (4-bit; 8-bit: M <= 8) with >= 512 tiles of 16 columns and 8
    or 16 groups takes the streaming GEMV for 2-byte types (one 16-row MFMA
    tile, A rows past M clamped; 515 tiles: two column tiles per wave at
    M = 5..8, four at M = 9..16, the last workgroup's tiles partly or wholly
    past N), 8-bit at 9 <= M <= 16 the mid-M launch, fp32 the workgroup-fold
    GEMV: rows equal the oracle bit for bit and the same rows computed alone,
    bit for bit."""
    N, K = 8192 + 40, 4096     # 515 column tiles, the last one partial; G = 16
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 3 + gs)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((16, K), DT[dt], gen(13))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    W = ora.dequantize(wq.cpu().view(torch.int32).numpy().view(np.uint32), to_np(s.cpu()), to_np(b.cpu()),
                       gs, bits_, dt)
    cols = np.r_[0:24, 4100:4124, N - 24:N]
    for M in (1, 2, 4, 5, 8, 9, 12, 16):
        got = run(x[:M])
        rows = sorted({0, M // 2, M - 1})
        want = ora.matmul(to_np(x[rows]), W[cols], dt, kmap="blocked")
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"{dt} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (4, 128)])
@pytest.mark.parametrize("N,K", [(2048 + 40, 4096), (4096 + 24, 8192), (4096 + 8, 14336), (16, 4096), (1000, 2048),
                                 (200, 1024)])
def test_quantized_stream_launch_fewer_tiles_and_longer_k(bits_, gs, N, K):
    """The streaming GEMV below 512 column tiles (131, 258 and 63 tiles, the
    last one partial, and a single tile), at 32 and 56 groups (eight and
    fourteen waves of four groups) and at 4 groups (M <= 2 with groups of up
    to 64 only): M <= 16 (4-bit) / 8 (8-bit) where A's rows fit in LDS; past
    that (32 groups: M > 8, 56 groups: M > 4) with A read per group from
    global memory at 258 / 257 tiles, the mid-M launch or the workgroup-fold
    GEMV at fewer. Rows equal the oracle and the same rows computed alone, bit
    for bit."""
    dt = "bf16"
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 11 + gs + K % 977)
    cols = np.unique(np.clip(np.r_[0:24, N // 2:N // 2 + 16, N - 24:N], 0, N - 1))
    W = ora.dequantize(wq[cols].view(torch.int32).numpy().view(np.uint32), to_np(s[cols]), to_np(b[cols]),
                       gs, bits_, dt)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((16, K), DT[dt], gen(19))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    for M in (1, 2, 3, 5, 8, 12, 16):
        got = run(x[:M])
        rows = sorted({0, M // 2, M - 1})
        want = ora.matmul(to_np(x[rows]), W, dt, kmap="blocked")
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (8, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantized_stream_a_from_global(bits_, gs, dt):
    """5 <= M <= 16 where A's rows x K do not fit in LDS (56 groups at M > 4,
    32 groups at M > 8; 8-bit codes up to 16 rows as well) with at least 256
    column tiles: the streaming GEMV with A's fragments read per group from
    global memory (7 waves of 8 groups at 56, 4 of 8 at 32), on exactly 256
    tiles and on 257 with the last one partial; 255 tiles take the launch
    before. x is a column slice of a wider matrix (row stride K + 64) whose
    rows past M hold other values. Rows equal the oracle and the same rows
    computed alone, bit for bit."""
    for N, K in ((4096, 14336), (4096 + 8, 8192), (4080, 14336)):
        wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 7 + gs + N % 97)
        cols = np.unique(np.clip(np.r_[0:16, N // 2:N // 2 + 8, N - 16:N], 0, N - 1))
        W = ora.dequantize(wq[cols].view(torch.int32).numpy().view(np.uint32), to_np(s[cols]), to_np(b[cols]),
                           gs, bits_, dt)
        wq, s, b = wq.cuda(), s.cuda(), b.cuda()
        xw = randn((17, K + 64), DT[dt], gen(K + bits_))
        run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
        for M in (5, 9, 16):
            x = xw[:M, 32:32 + K]
            assert x.stride(0) == K + 64
            got = run(x)
            rows = sorted({0, M // 2, M - 1})
            want = ora.matmul(to_np(x[rows]), W, dt, kmap="blocked")
            assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
            for rr in rows:
                assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1].contiguous())), (N, K, M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32)])
@pytest.mark.parametrize("N,K", [(1000, 14336), (2048, 8192), (520, 16384)])
def test_quantized_split_k_few_columns_long_k(bits_, gs, N, K):
    """5 <= M <= 16 with at most 2048 columns and 32 or more groups where the
    streaming GEMV does not take the shape (A's rows x K beyond LDS; 64
    groups): K split into chunks of 4 groups, the per-group partials folded in
    group order. Rows equal the oracle and the same rows computed alone (the
    streaming GEMV or the workgroup-fold GEMV), bit for bit."""
    dt = "bf16"
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 5 + gs + K % 1013)
    cols = np.unique(np.clip(np.r_[0:16, N // 2:N // 2 + 8, N - 16:N], 0, N - 1))
    W = ora.dequantize(wq[cols].view(torch.int32).numpy().view(np.uint32), to_np(s[cols]), to_np(b[cols]),
                       gs, bits_, dt)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((16, K), DT[dt], gen(23))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    for M in (5, 8, 12, 16):
        got = run(x[:M])
        rows = sorted({0, M - 1})
        want = ora.matmul(to_np(x[rows]), W, dt, kmap="blocked")
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantized_mid_m_split_k_matches_oracle(bits_, gs, dt):
    """Few column blocks (N = 4136: 65 blocks of 64) make the mid-M launch split
    K into chunks (15 groups: 8 chunks of 2, the last of 1) with per-group
    partials folded afterwards; M = 200 (four 64-row blocks, 260 tiles) runs
    unsplit. Rows equal the oracle and the same rows
    computed alone, bit for bit."""
    N, K = 4096 + 40, 15 * 256
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 5 + gs + 1)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    from mlx_batch_invariant_amd import _lib
    assert _lib.load().bi_quantized_matmul_workspace_bytes(64, N, K) == 15 * 64 * N * 4
    assert _lib.load().bi_quantized_matmul_workspace_bytes(200, N, K) == 0
    x = randn((200, K), DT[dt], gen(17))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    W = ora.dequantize(wq.cpu().view(torch.int32).numpy().view(np.uint32), to_np(s.cpu()), to_np(b.cpu()),
                       gs, bits_, dt)
    cols = np.r_[0:24, 2050:2074, N - 24:N]
    for M in (17, 33, 64, 200):
        got = run(x[:M])
        rows = sorted({0, M // 2, M - 1})
        want = ora.matmul(to_np(x[rows]), W[cols], dt, kmap="blocked")
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"{dt} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(run(x[rr:rr + 1])), (M, rr)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32), (8, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [800, 256])
def test_quantized_large_m_launch_agrees(bits_, gs, dt, M):
    """Large M takes the dequantize-once launch (weights dequantized into the
    workspace in the dense tile's k order, then the large dense tile: 4 x 112
    tiles of 256 x 128 at M = 800, 2 x 112 of 128 x 128 at M = 256): its rows
    equal the same rows computed alone (M = 1, the GEMV launch) bit for bit,
    and the oracle bit for bit."""
    N, K = 14336, 1024
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ + gs + 5)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    from mlx_batch_invariant_amd import _lib
    assert _lib.load().bi_quantized_matmul_workspace_bytes(M, N, K) == (N + M) * K * 2
    x = randn((M, K), DT[dt], gen(21))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    full = run(x)
    rows = [0, min(257, M - 2), M - 1]
    for rr in rows:
        assert bits(full[rr:rr + 1]) == bits(run(x[rr:rr + 1])), rr
    W = ora.dequantize(wq.cpu().view(torch.int32).numpy().view(np.uint32), to_np(s.cpu()), to_np(b.cpu()),
                       gs, bits_, dt)
    cols = np.r_[0:32, 7000:7032, N - 32:N]
    want = ora.matmul(to_np(x[rows]), W[cols], dt, kmap="blocked")
    assert_bits_equal(to_np(full)[rows][:, cols], want, f"{dt} large M")


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128)])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (4096, 14336)])
def test_quantized_prefill_m512_launch_agrees(bits_, gs, N, K):
    """Config-5 prefill at B = 1 (M = 512) at the Llama projection shapes:
    the weight dequantized once into the workspace, then the dense policy's
    launch (the 128 x 64 large tile for N = 4096, the unsplit tall tile for
    N = 1024). Sampled rows equal the same rows computed alone (the GEMV) and
    the oracle, bit for bit."""
    M = 512
    from mlx_batch_invariant_amd import _lib
    assert _lib.load().bi_quantized_matmul_workspace_bytes(M, N, K) == (N + M) * K * 2
    wq, s, b = _qweights(N, K, bits_, gs, "bf16", seed=bits_ + N + K)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    x = randn((M, K), torch.bfloat16, gen(N + K))
    run = lambda xx: _bi().batch_invariant_quantized_matmul(xx, wq, s, b, group_size=gs, bits=bits_)
    got = run(x)
    W = ora.dequantize(wq.cpu().view(torch.int32).numpy().view(np.uint32), to_np(s.cpu()), to_np(b.cpu()),
                       gs, bits_, "bf16")
    rows = [0, 127, 128, 300, 511]
    cols = np.r_[0:24, N // 2:N // 2 + 24, N - 24:N]
    want = ora.matmul(to_np(x[rows]), W[cols], "bf16", kmap="blocked")
    assert_bits_equal(to_np(got)[rows][:, cols], want, f"M=512 N={N} K={K}")
    for r in rows:
        assert bits(got[r:r + 1]) == bits(run(x[r:r + 1])), r


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32)])
def test_quantized_batch_invariant_llama_mlp(bits_, gs):
    """W [14336, 4096], x [M, 4096], M in 1..64 (and beyond)."""
    N, K = 14336, 4096
    wq, s, b = _qweights(N, K, bits_, gs, "bf16", seed=0)
    wq, s, b = wq.cuda(), s.cuda(), b.cuda()
    probe = randn((1, K), torch.bfloat16, gen(1))
    run = lambda x: _bi().batch_invariant_quantized_matmul(x, wq, s, b, group_size=gs, bits=bits_)
    fails = sweep(probe, lambda n, gg: randn((n, K), torch.bfloat16, gg), run,
                  batches=[1, 2, 4, 8, 16, 32, 64, 128, 256])
    assert not fails, fails


def test_quantized_errors():
    bi = _bi()
    x = torch.zeros((2, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((8, 8), dtype=torch.uint32, device="cuda")
    s = torch.zeros((8, 1), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        bi.batch_invariant_quantized_matmul(x, w, s, s, group_size=64, bits=3)
    with pytest.raises(ValueError):
        bi.batch_invariant_quantized_matmul(x[:, :32], w, s, s, group_size=64, bits=4)


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 128), (4, 32)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dequantized_once_equals_the_quantized_op(bits_, gs, dt):
    """bi_quantized_matmul_dequantized on the weight dequantized once
    (bi_quantized_dequantize) equals bi_quantized_matmul bit for bit at every M
    (the GEMV, mid-M and large-M launches of the quantized op against the
    dense launches on the reordered operands); the cache that
    batch_invariant_quantized_matmul uses from DEQUANTIZED_MIN_M rows gives the
    same bits, follows only the cached tensors, and is released by
    drop_dequantized."""
    from mlx_batch_invariant_amd import _lib
    from mlx_batch_invariant_amd.kernels import quantized as kq
    bi = _bi()
    N, K = 1000, 768
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 13 + gs)
    wq, s, b = wq.view(torch.int32).cuda(), s.cuda(), b.cuda()
    x = randn((300, K), DT[dt], gen(23))
    lib = _lib.load()
    bq = torch.empty((N, K), dtype=DT[dt], device="cuda")
    _lib.check(lib.bi_quantized_dequantize(wq.data_ptr(), s.data_ptr(), b.data_ptr(), bq.data_ptr(), N, K, bits_, gs,
                                           _lib.DTYPE_CODE[DT[dt]], None), "bi_quantized_dequantize")
    for M in (1, 5, 16, 64, 255, 256, 300):
        want = bi.batch_invariant_quantized_matmul(x[:M], wq, s, b, group_size=gs, bits=bits_)
        need = lib.bi_quantized_matmul_dequantized_workspace_bytes(M, N, K)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        got = torch.empty((M, N), dtype=DT[dt], device="cuda")
        _lib.check(lib.bi_quantized_matmul_dequantized(x.data_ptr(), x.stride(0), bq.data_ptr(), got.data_ptr(), M, N,
                                                       K, _lib.DTYPE_CODE[DT[dt]], ws.data_ptr(), need, None),
                   "bi_quantized_matmul_dequantized")
        torch.cuda.synchronize()
        assert bits(got) == bits(want), M
    # the cache inside batch_invariant_quantized_matmul
    plain = bi.batch_invariant_quantized_matmul(x, wq, s, b, group_size=gs, bits=bits_)
    cached = bi.cache_dequantized(wq, s, b, group_size=gs, bits=bits_)
    assert bits(cached) == bits(bq)
    assert kq._dequantized_for(wq, s, b, gs, bits_, DT[dt]) is not None
    assert kq._dequantized_for(wq, s.clone(), b, gs, bits_, DT[dt]) is None      # other scales: not this copy
    assert bits(bi.batch_invariant_quantized_matmul(x, wq, s, b, group_size=gs, bits=bits_)) == bits(plain)
    assert bits(bi.batch_invariant_quantized_matmul(x[:16], wq, s, b, group_size=gs, bits=bits_)) == bits(plain[:16])
    bi.drop_dequantized(wq)
    assert kq._dequantized_for(wq, s, b, gs, bits_, DT[dt]) is None


def test_quantized_linear_cache_under_the_mode():
    """QuantizedLinear.cache_dequantized: the module's prefill-sized call under
    the mode gives the same bits with and without the cached copy."""
    bi = _bi()
    from mlx_batch_invariant_amd.nn import QuantizedLinear
    lin = torch.nn.Linear(1024, 2048, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn((2048, 1024), generator=gen(29)) * 0.02)
    q = QuantizedLinear.from_linear(lin.to(torch.bfloat16), group_size=64, bits=4).cuda()
    x = randn((2, 300, 1024), torch.bfloat16, gen(31))
    with bi.set_batch_invariant_mode(strict=True):
        plain = q(x)
        q.cache_dequantized()
        cached = q(x)
    assert bits(cached) == bits(plain)
    bi.drop_dequantized(q.weight)


def _pack_reference(wq, s, b, bits_, gs, N, K):
    """numpy restatement of bi_quantized_pack's layout (the QuantPacked
    source of the streaming GEMV): block (tile t, group g) of bits x 512 +
    16 x (256 / gs) x 4 bytes holds, for MFMA lane l = r + 16 q (row
    min(16 t + r, N - 1), k [256 g + 64 q, +64)), its 64 x bits / 32 code
    words as 16-byte pieces at 1024 i + 16 l, then the block's (scale, bias)
    pairs (16-bit each, scale low), each once: lane l's P pairs (P = 2 for
    group size 32, else 1; pair i of group k0 / gs + i) at bits x 512 +
    4 (P l + i) for groups of 32 and 64, row r's pair of 128-k half h at
    bits x 512 + 4 (16 h + r) for groups of 128."""
    words = wq.cpu().view(torch.int32).numpy().view(np.uint32)
    sb = s.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32)
    bb = b.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32)
    G, tiles, pieces = K // 256, (N + 15) // 16, bits_ // 2
    pairs = 2 if gs == 32 else 1
    wpl = 64 * bits_ // 32                                   # words per lane and group
    blk = bits_ * 512 + 16 * (256 // gs) * 4
    out = np.zeros(tiles * G * blk, np.uint8)
    for t in range(tiles):
        for g in range(G):
            base = (t * G + g) * blk
            for lane in range(64):
                r, q = lane % 16, lane // 16
                n = min(16 * t + r, N - 1)
                k0 = 256 * g + 64 * q
                wv = words[n, k0 * bits_ // 32:k0 * bits_ // 32 + wpl]
                for i in range(pieces):
                    o = base + 1024 * i + 16 * lane
                    out[o:o + 16] = wv[4 * i:4 * i + 4].view(np.uint8)
                for i in range(pairs):
                    m = np.uint32(sb[n, k0 // gs + i] | (bb[n, k0 // gs + i] << 16))
                    slot = 16 * (q * 64 // gs) + r if gs == 128 else pairs * lane + i
                    o = base + pieces * 1024 + 4 * slot
                    out[o:o + 4] = np.array([m], np.uint32).view(np.uint8)
    return out


@pytest.mark.parametrize("bits_,gs", [(4, 64), (8, 64), (4, 32), (8, 32), (4, 128), (8, 128)])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantized_pack_layout(bits_, gs, dt):
    """bi_quantized_pack writes exactly the layout restated in numpy above
    (20 rows: the second tile's rows past N repeat row N - 1; two groups)."""
    from mlx_batch_invariant_amd import _lib
    N, K = 20, 512
    wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ + gs + 41)
    lib = _lib.load()
    nbytes = lib.bi_quantized_pack_bytes(N, K, bits_, gs)
    got = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")
    wd, sd, bd = wq.cuda(), s.cuda(), b.cuda()      # held until the kernel has run
    _lib.check(lib.bi_quantized_pack(wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), got.data_ptr(), nbytes, N, K,
                                     bits_, gs, _lib.DTYPE_CODE[DT[dt]], None), "bi_quantized_pack")
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), _pack_reference(wq, s, b, bits_, gs, N, K))


@pytest.mark.parametrize("bits_,gs,dt", [(4, 64, "bf16"), (4, 64, "f16"), (8, 64, "bf16"), (8, 64, "f16"),
                                         (4, 32, "bf16"), (4, 128, "f16"), (8, 128, "bf16"), (8, 32, "f16")])
def test_quantized_packed_equals_the_quantized_op(bits_, gs, dt):
    """bi_quantized_matmul_packed with the repacked copy equals
    bi_quantized_matmul bit for bit at every M and group count: the streaming
    GEMV on the copy (16 groups at 131, 257 and 515 column tiles, the last one
    partial: 8 waves of 2 groups, or 16 of 1 with one, two or four column
    tiles per wave, at 257 tiles from one row; 8 groups; 4 groups at M <= 2; 32 and 56 groups, A staged
    or read from global memory at 257 and 258 tiles), the mid-M launches on
    the copy (M = 20 .. 100; 33 .. 64 rows on 65 and 129 column blocks as
    unsplit 32-row blocks; 5 .. 16 rows split over K with 1000 columns and 56
    groups), and the MLX-layout launches where neither takes the shape
    (12 groups at M <= 16; 4 groups at M > 2). The cache
    inside batch_invariant_quantized_matmul (up to PACKED_MAX_M rows) gives the
    same bits, follows only the cached tensors, and is released by
    drop_packed."""
    from mlx_batch_invariant_amd import _lib
    from mlx_batch_invariant_amd.kernels import quantized as kq
    bi = _bi()
    lib = _lib.load()
    code = _lib.DTYPE_CODE[DT[dt]]
    for N, K in ((2048 + 40, 4096), (4096 + 8, 4096), (8192 + 40, 4096), (1000, 2048), (100, 1024),
                 (4096 + 8, 14336), (4096 + 24, 8192), (300, 3072), (1000, 14336)):
        wq, s, b = _qweights(N, K, bits_, gs, dt, seed=bits_ * 17 + gs + N % 89 + K % 97)
        wq, s, b = wq.view(torch.int32).cuda(), s.cuda(), b.cuda()
        nbytes = lib.bi_quantized_pack_bytes(N, K, bits_, gs)
        bp = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
        _lib.check(lib.bi_quantized_pack(wq.data_ptr(), s.data_ptr(), b.data_ptr(), bp.data_ptr(), nbytes, N, K,
                                         bits_, gs, code, None), "bi_quantized_pack")
        x = randn((100, K), DT[dt], gen(K + N))
        for M in (1, 2, 3, 5, 8, 12, 16, 20, 33, 64, 100):
            want = bi.batch_invariant_quantized_matmul(x[:M], wq, s, b, group_size=gs, bits=bits_)
            need = lib.bi_quantized_matmul_workspace_bytes(M, N, K)
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
            got = torch.empty((M, N), dtype=DT[dt], device="cuda")
            _lib.check(lib.bi_quantized_matmul_packed(x.data_ptr(), x.stride(0), wq.data_ptr(), s.data_ptr(),
                                                      b.data_ptr(), bp.data_ptr(), got.data_ptr(), M, N, K, bits_,
                                                      gs, code, ws.data_ptr(), need, None),
                       "bi_quantized_matmul_packed")
            torch.cuda.synchronize()
            assert bits(got) == bits(want), (N, K, M)
    # the cache inside batch_invariant_quantized_matmul (last shape's operands)
    plain = bi.batch_invariant_quantized_matmul(x, wq, s, b, group_size=gs, bits=bits_)
    cached = bi.cache_packed(wq, s, b, group_size=gs, bits=bits_)
    assert bits(cached) == bits(bp)
    assert kq._cached_for(kq._PACKED, wq, s, b, gs, bits_, DT[dt]) is not None
    assert kq._cached_for(kq._PACKED, wq, s.clone(), b, gs, bits_, DT[dt]) is None   # other scales: not this copy
    for M in (1, 7, 16, 20, 64, 100):
        assert bits(bi.batch_invariant_quantized_matmul(x[:M], wq, s, b, group_size=gs, bits=bits_)) == \
            bits(plain[:M]), M
    bi.drop_packed(wq)
    assert kq._cached_for(kq._PACKED, wq, s, b, gs, bits_, DT[dt]) is None


def test_quantized_linear_packed_under_the_mode():
    """QuantizedLinear.cache_packed: decode-sized calls under the mode give the
    same bits with and without the repacked copy, and the copy is used."""
    bi = _bi()
    from mlx_batch_invariant_amd.kernels import quantized as kq
    from mlx_batch_invariant_amd.nn import QuantizedLinear
    lin = torch.nn.Linear(4096, 1024, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn((1024, 4096), generator=gen(37)) * 0.02)
    q = QuantizedLinear.from_linear(lin.to(torch.bfloat16), group_size=64, bits=4).cuda()
    x = randn((4, 3, 4096), torch.bfloat16, gen(43))
    with bi.set_batch_invariant_mode(strict=True):
        plain = [q(x[:, :t]) for t in (1, 2, 3)]
        q.cache_packed()
        assert kq._cached_for(kq._PACKED, q.weight, q.scales, q.biases, 64, 4, torch.bfloat16) is not None
        cached = [q(x[:, :t]) for t in (1, 2, 3)]
    for p_, c_ in zip(plain, cached):
        assert bits(c_) == bits(p_)
    bi.drop_packed(q.weight)
