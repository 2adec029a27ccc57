"""Dense matmul on the GPU: integer known answers (exact), identity, bitwise
parity with the oracle (which models the gfx950 MFMA accumulation exactly),
batch invariance across the split/fused and tile-height boundaries, MFMA row
independence."""

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, bits, gen, randn, to_np
from oracle import bi_oracle as ora
from sweep import sweep

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _mm(a, b):
    return _bi().batch_invariant_matmul(a, b)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (5, 100, 896), (33, 48, 1000), (100, 130, 512), (17, 16, 8), (300, 70, 264)])
def test_matmul_integer_known_answer(dt, M, N, K):
    """Small integers: every partial sum is an integer < 2^24, so every order is
    exact and the result must equal the int64 product bit for bit."""
    rng = np.random.default_rng(M * 1000 + N + K)
    a = rng.integers(-3, 4, size=(M, K))
    bt = rng.integers(-3, 4, size=(N, K))
    want = a @ bt.T
    assert np.abs(want).max() < 2 ** 24  # the fp32 total is the exact integer
    A = torch.tensor(a, dtype=DT[dt]).cuda()
    Bt = torch.tensor(bt, dtype=DT[dt]).cuda()
    got = _mm(A, Bt.t())
    np.testing.assert_array_equal(to_np(got), ora.round_to(want.astype(np.float32), dt))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_matmul_identity(dt):
    g = gen(3)
    K = 640
    Bt = randn((96, K), DT[dt], g)
    eye = torch.eye(K, dtype=DT[dt]).cuda()
    got = _mm(eye, Bt.t())                  # row k of the result is column k of B
    assert bits(got) == bits(Bt.t().contiguous())


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M,N,K", [(1, 4864, 896), (16, 256, 4096), (32, 200, 896), (64, 300, 1024), (257, 130, 520),
                                   (16, 64, 65 * 256)])
def test_matmul_matches_oracle(dt, M, N, K):
    """Every launch shape (GEMV, workgroup fold, split partials + fold kernel,
    mid-M tall tile, LDS tiles) against the oracle, bit for bit (fp16 weights
    at scale 0.02 include subnormal operands)."""
    g = gen(M + N + K)
    a = randn((M, K), DT[dt], g)
    bt = randn((N, K), DT[dt], g, scale=0.02)
    got = to_np(_mm(a, bt.t()))
    assert_bits_equal(got, ora.matmul(to_np(a), to_np(bt), dt), f"{dt} {M}x{N}x{K}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_matmul_wide_range_operands_match_oracle(dt):
    """Operands spread over many binades (products far apart, heavy truncation
    and cancellation inside the MFMA blocks): still bit for bit."""
    rng = np.random.default_rng(11)
    lo, hi = (-12, 12) if dt == "bf16" else (-6, 6)
    a = rng.standard_normal((20, 2048)) * np.exp2(rng.integers(lo, hi, (20, 2048)))
    bt = rng.standard_normal((96, 2048)) * np.exp2(rng.integers(lo, hi, (96, 2048)))
    A = torch.tensor(a, dtype=torch.float32).to(DT[dt]).cuda()
    Bt = torch.tensor(bt, dtype=torch.float32).to(DT[dt]).cuda()
    assert_bits_equal(to_np(_mm(A, Bt.t())), ora.matmul(to_np(A), to_np(Bt), dt), dt)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("N,K", [(4864, 896), (4096, 4096)])
def test_matmul_batch_invariant(dt, N, K):
    g = gen(0)
    W = randn((N, K), DT[dt], g, scale=0.02)
    probe = randn((1, K), DT[dt], g)
    fails = sweep(probe, lambda n, gg: randn((n, K), DT[dt], gg), lambda x: _mm(x, W.t()))
    assert not fails, fails


def test_matmul_row_position_independence():
    """The probe row at every position of 16- and 64-row batches: MFMA rows are
    computed independently of the other rows of the tile."""
    g = gen(5)
    K, N = 1024, 256
    W = randn((N, K), torch.bfloat16, g, scale=0.02)
    probe = randn((1, K), torch.bfloat16, g)
    fails = sweep(probe, lambda n, gg: randn((n, K), torch.bfloat16, gg), lambda x: _mm(x, W.t()),
                  batches=[16, 64, 48], positions=lambda B: range(B))
    assert not fails, fails


@pytest.mark.parametrize("K", [4096, 65 * 256 + 128])
def test_matmul_launch_shapes_agree(K):
    """M = 1, 16 (the streaming GEMV at 16 groups; split partials + fold
    kernel at 66 groups), 17..32 (two m-tiles) and 33 (LDS tiles, register
    fold) give the same bits for the same rows."""
    g = gen(6)
    N = 160
    W = randn((N, K), torch.bfloat16, g, scale=0.02)
    x = randn((33, K), torch.bfloat16, g)
    fused = _mm(x, W.t())
    for M in (1, 16, 20, 32):
        assert bits(_mm(x[:M], W.t())) == bits(fused[:M]), M


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("K", [512, 4096])
def test_matmul_large_tiles_agree(dt, K):
    """Large M x N (the 256 x 128 direct-to-LDS tile; partial last tiles in
    both m and n) gives the decode launches' bits for the same rows, and
    matches the oracle on a sample of rows."""
    g = gen(9)
    M, N = 2100, 4136                      # 9 x 33 tiles of 256 x 128
    W = randn((N, K), DT[dt], g, scale=0.02)
    x = randn((M, K), DT[dt], g)
    big = _mm(x, W.t())
    for lo, hi in ((0, 1), (255, 256), (256, 272), (2099, 2100), (1000, 1032)):
        assert bits(_mm(x[lo:hi], W.t())) == bits(big[lo:hi]), (lo, hi)
    rows = [0, 1, 255, 256, 1337, 2048, 2099]
    assert_bits_equal(to_np(big[rows]), ora.matmul(to_np(x[rows]), to_np(W), dt), f"{dt} K={K}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("K", [512, 4096])
def test_matmul_large_half_tiles_agree(dt, K):
    """The large tile run as 128 x 128 tiles (its 256-row tiles would leave CUs
    idle; partial last tiles in both m and n) gives the decode launches' bits
    for the same rows and matches the oracle on a sample of rows."""
    from mlx_batch_invariant_amd import _lib
    M, N = 200, 12400                      # 2 x 97 tiles of 128 x 128
    assert _lib.load().bi_matmul_launch(M, N, K) == b"big 128x128"
    g = gen(10)
    W = randn((N, K), DT[dt], g, scale=0.02)
    x = randn((M, K), DT[dt], g)
    big = _mm(x, W.t())
    for lo, hi in ((0, 1), (127, 128), (128, 144), (199, 200), (60, 92)):
        assert bits(_mm(x[lo:hi], W.t())) == bits(big[lo:hi]), (lo, hi)
    rows = [0, 1, 127, 128, 150, 199]
    assert_bits_equal(to_np(big[rows]), ora.matmul(to_np(x[rows]), to_np(W), dt), f"{dt} K={K}")


@pytest.mark.parametrize("M,N,K,launch", [(80, 14336, 4096, "big 128x64"), (128, 14336, 4096, "big 128x64"),
                                          (128, 4864, 896, "big 128x64"), (512, 4096, 4096, "big 128x64"),
                                          (512, 4096, 14336, "big 128x64"), (768, 4096, 4096, "big 128x128"),
                                          (768, 1024, 4096, "big 128x64"), (512, 1024, 4096, "tall 32x32 k128 r4 c1"),
                                          (384, 896, 4864, "tall 32x32 k128 r4 c1")])
def test_matmul_mid_m_large_tile_forms(M, N, K, launch):
    """The 128 x 64 and 128 x 128 large-tile forms and the tall tile above
    M = 256 at the Llama / Qwen2 shapes that select them (config-5 prefill at
    B = 1 is M = 512): sampled rows (first, last, both sides of the 128-row
    tile edge) equal the same rows computed alone (the decode launches) and
    the oracle on a column sample, bit for bit."""
    lib = _bi()._lib.load()
    assert lib.bi_matmul_launch(M, N, K).decode() == launch
    g = gen(M + N + 3 * K)
    W = randn((N, K), torch.bfloat16, g, scale=0.02)
    x = randn((M, K), torch.bfloat16, g)
    full = _mm(x, W.t())
    rows = sorted(r for r in {0, 1, 63, 64, 127, 128, M // 2, M - 1} if r < M)   # in range for every M
    cols = np.r_[0:32, 60:70, N // 2:N // 2 + 32, N - 32:N]
    want = ora.matmul(to_np(x[rows]), to_np(W)[cols], "bf16")
    assert_bits_equal(to_np(full)[rows][:, cols], want, launch)
    for r in rows:
        assert bits(_mm(x[r:r + 1], W.t())) == bits(full[r:r + 1]), r
    assert bits(_mm(x[M - 40:], W.t())) == bits(full[M - 40:])


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("N,K", [(2048 + 40, 4096), (4096 + 8, 14336), (4096, 2048), (8192 + 24, 8192), (16, 4096),
                                 (1000, 2048), (5, 8192), (40, 14336)])
def test_matmul_stream_launch_matches_oracle(dt, N, K):
    """M <= 16 with 8 / 16 / 32 / 56 groups takes the streaming GEMV for a
    dense B at any number of column tiles (one tile, a single partial tile of
    5 columns, 63 with the last partial, up to 515; A's rows staged per wave
    in LDS; 32 groups: M <= 8, 56 groups: M <= 4; past that A read per group
    from global memory at 257 and 515 tiles, the workgroup-fold GEMV at
    fewer): rows equal the oracle and the same rows computed alone, bit for
    bit."""
    g = gen(N + K)
    bt = randn((N, K), DT[dt], g)
    x = randn((16, K), DT[dt], g)
    cols = np.unique(np.clip(np.r_[0:24, N // 2:N // 2 + 16, N - 24:N], 0, N - 1))
    W = to_np(bt[cols])
    for M in (1, 3, 5, 8, 12, 16):
        got = _mm(x[:M], bt.t())
        rows = sorted({0, M // 2, M - 1})
        want = ora.matmul(to_np(x[rows]), W, dt)
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(_mm(x[rr:rr + 1], bt.t())), (M, rr)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_matmul_stream_a_from_global(dt):
    """5 <= M <= 16 where A's rows x K do not fit in LDS (56 groups at M > 4,
    32 groups at M > 8) with at least 256 column tiles: the dense streaming
    GEMV with A's fragments read per group from global memory (7 waves of 8
    groups at 56, 8 of 4 at 32), on exactly 256 tiles and on 257 with the
    last one partial; 255 tiles take the launch before. x is a column slice
    of a wider matrix (row stride K + 64). Rows equal the oracle and the same
    rows computed alone, bit for bit."""
    for N, K in ((4096, 14336), (4096 + 8, 8192), (4080, 14336)):
        g = gen(N + 5 * K)
        bt = randn((N, K), DT[dt], g)
        xw = randn((17, K + 64), DT[dt], g)
        cols = np.unique(np.clip(np.r_[0:16, N // 2:N // 2 + 8, N - 16:N], 0, N - 1))
        W = to_np(bt[cols])
        for M in (5, 9, 16):
            x = xw[:M, 32:32 + K]
            assert x.stride(0) == K + 64
            got = _mm(x, bt.t())
            rows = sorted({0, M // 2, M - 1})
            want = ora.matmul(to_np(x[rows]), W, dt)
            assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
            for rr in rows:
                assert bits(got[rr:rr + 1]) == bits(_mm(x[rr:rr + 1].contiguous(), bt.t())), (N, K, M, rr)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("N,K", [(1000, 14336), (2048, 8192), (520, 16384)])
def test_matmul_split_k_few_columns_long_k(dt, N, K):
    """5 <= M <= 16 with at most 2048 columns and 32 or more groups where the
    dense streaming GEMV does not take the shape (A's rows x K beyond LDS; 64
    groups): the mid-M tile on a dense B with K split into chunks of 4
    groups, the per-group partials folded in group order. Rows equal the
    oracle and the same rows computed alone, bit for bit."""
    g = gen(N + 3 * K)
    bt = randn((N, K), DT[dt], g)
    x = randn((16, K), DT[dt], g)
    cols = np.unique(np.clip(np.r_[0:16, N // 2:N // 2 + 8, N - 16:N], 0, N - 1))
    W = to_np(bt[cols])
    for M in (5, 8, 12, 16):
        got = _mm(x[:M], bt.t())
        rows = sorted({0, M - 1})
        want = ora.matmul(to_np(x[rows]), W, dt)
        assert_bits_equal(to_np(got)[rows][:, cols], want, f"N={N} K={K} M={M}")
        for rr in rows:
            assert bits(got[rr:rr + 1]) == bits(_mm(x[rr:rr + 1], bt.t())), (M, rr)


def test_matmul_layouts_and_leading_dims():
    g = gen(7)
    a = randn((2, 3, 200), torch.bfloat16, g)
    b_row = randn((200, 72), torch.bfloat16, g)      # row-major [K, N]: copied to k-major
    out = _mm(a, b_row)
    ref = _mm(a.reshape(6, 200), b_row.t().contiguous().t())
    assert out.shape == (2, 3, 72)
    assert bits(out.reshape(6, 72)) == bits(ref)
    v = randn((200,), torch.bfloat16, g)             # 1-D lhs
    assert _mm(v, b_row).shape == (72,)
    odd = randn((3, 13), torch.float16, g)           # K % 8 != 0 -> zero-padded copy
    w13 = randn((13, 5), torch.float16, g)
    assert_bits_equal(to_np(_mm(odd, w13)), ora.matmul(to_np(odd), to_np(w13).T, "f16"), "K=13")


def test_matmul_errors():
    bi = _bi()
    a = torch.zeros((2, 8), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        bi.batch_invariant_matmul(a, torch.zeros((9, 4), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        bi.batch_invariant_matmul(a, torch.zeros((2, 8, 4), dtype=torch.bfloat16, device="cuda"))
    assert bi.batch_invariant_matmul(a[:0], torch.zeros((8, 4), dtype=torch.bfloat16, device="cuda")).shape == (0, 4)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("ashape,bshape,trans", [((3, 40, 256), (3, 256, 100), False),
                                                 ((2, 1, 17, 96), (5, 96, 33), False),
                                                 ((4, 33, 128), (4, 70, 128), True),
                                                 ((40, 512), (3, 512, 64), False)])
def test_batched_matmul_slices_equal_2d_calls(dt, ashape, bshape, trans):
    """Every slice of the batched launch is the 2-D kernel on that slice (bits),
    with broadcast batch dims and a transposed right-hand side (q @ k^T)."""
    bi = _bi()
    g = gen(sum(ashape) + sum(bshape))
    a = randn(ashape, DT[dt], g)
    b = randn(bshape, DT[dt], g)
    if trans:
        b = b.transpose(-1, -2)                   # [..., K, N] view of a k-contiguous [..., N, K]
    got = bi.batch_invariant_bmm(a, b)
    batch = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    assert tuple(got.shape) == (*batch, a.shape[-2], b.shape[-1])
    ae = a.expand(*batch, *a.shape[-2:])
    be = b.expand(*batch, *b.shape[-2:])
    for idx in np.ndindex(*batch):
        assert bits(got[idx]) == bits(bi.batch_invariant_matmul(ae[idx], be[idx])), idx
    i0 = (0,) * len(batch)
    assert_bits_equal(to_np(got[i0]), ora.matmul(to_np(ae[i0]), to_np(be[i0]).T, dt), dt)


def test_batched_matmul_rows_independent_of_m_and_batch():
    bi = _bi()
    g = gen(8)
    a = randn((6, 64, 1024), torch.bfloat16, g)
    b = randn((6, 1024, 300), torch.bfloat16, g)
    full = bi.batch_invariant_bmm(a, b)
    for m in (1, 16, 33):
        assert bits(bi.batch_invariant_bmm(a[:, :m], b)) == bits(full[:, :m]), m
    assert bits(bi.batch_invariant_bmm(a[2:3], b[2:3])) == bits(full[2:3])


def test_batched_matmul_intercepted_by_mode():
    bi = _bi()
    g = gen(9)
    q = randn((2, 4, 16, 64), torch.bfloat16, g)
    k = randn((2, 4, 40, 64), torch.bfloat16, g)
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        s1 = torch.matmul(q, k.transpose(-1, -2))
        s2 = q @ k.transpose(-1, -2)
        s3 = torch.bmm(q[0], k[0].transpose(-1, -2))
    assert bi.stats()["handled"] == {"matmul": 3}
    assert bits(s1) == bits(s2) == bits(bi.batch_invariant_bmm(q, k.transpose(-1, -2)))
    assert bits(s3) == bits(s1[0])


@pytest.mark.parametrize("M,N,K", [(200, 4864, 896), (256, 4864, 896), (160, 1024, 4096), (129, 12800, 896),
                                   (300, 12416, 960), (256, 4096, 4096)])
def test_matmul_m_above_128_and_partial_groups(M, N, K):
    """M > 128: the 256 x 128 tile where it has >= 96 tiles (M > 256: also
    >= 32 with at most 4 groups of K), the tall tile otherwise; K need not be
    whole groups (stages past K are zero). Sampled rows equal the oracle and
    the same rows computed alone, bit for bit (the decode launches)."""
    g = gen(M + N + K)
    W = randn((N, K), torch.bfloat16, g, scale=0.02)
    x = randn((M, K), torch.bfloat16, g)
    full = _mm(x, W.t())
    rows = sorted({0, 1, 127, 128, M // 2, M - 1})
    cols = np.r_[0:40, N // 2:N // 2 + 40, N - 40:N]
    want = ora.matmul(to_np(x[rows]), to_np(W)[cols], "bf16")
    assert_bits_equal(to_np(full)[rows][:, cols], want, f"{M}x{N}x{K}")
    for lo, hi in ((0, 1), (M - 1, M), (5, 21), (100, 164)):
        assert bits(_mm(x[lo:hi], W.t())) == bits(full[lo:hi]), (lo, hi)


TALL = [(40, 256, 640, "tall 32x32 k128 r4 c1"), (20, 256, 640, "tall 32x32 k128 r4 c3"),
        (20, 6400, 640, "tall 32x64 k128 r4 c1"), (256, 2304, 640, "tall 64x32 k128 r3 c1"),
        (200, 768, 2048, "tall 64x32 k128 r3 c4"), (256, 4352, 576, "tall 64x32 k64 r4 c1"),
        (200, 1280, 1984, "tall 64x32 k64 r4 c4"), (200, 6400, 576, "tall 64x64 k64 r4 c1"),
        (256, 3328, 576, "tall 32x64 k64 r5 c1"), (200, 1024, 1984, "tall 32x64 k64 r5 c4"),
        (40, 256, 576, "tall 32x32 k64 r6 c1"), (20, 256, 832, "tall 32x32 k64 r6 c4")]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,N,K,launch", TALL, ids=[t[3].replace(" ", "_") for t in TALL])
def test_matmul_tall_configurations(dt, M, N, K, launch):
    """Every configuration of the dense mid-M tile (tile, k per stage, ring
    depth; unsplit and with K in chunks + the ordered fold), picked by the
    policy at these shapes: sampled rows equal the oracle and the same rows
    computed alone (the decode launches), bit for bit."""
    lib = _bi()._lib.load()
    assert lib.bi_matmul_launch(M, N, K).decode() == launch
    g = gen(M * 7 + N + K)
    W = randn((N, K), DT[dt], g, scale=0.02)
    x = randn((M, K), DT[dt], g)
    full = _mm(x, W.t())
    rows = sorted({0, 15, 16, 31, 32, M // 2, M - 1} & set(range(M)))
    assert_bits_equal(to_np(full)[rows], ora.matmul(to_np(x[rows]), to_np(W), dt), f"{dt} {launch}")
    for lo, hi in ((0, 1), (M - 1, M), (3, 19)):
        assert bits(_mm(x[lo:hi], W.t())) == bits(full[lo:hi]), (lo, hi)


def _dense_pack_reference(bt, N, K):
    """numpy restatement of bi_matmul_pack's layout (the DensePacked source of
    the streaming GEMV): block (tile t, group g < ceil(K / 256)) of 8 KB holds,
    for MFMA lane l = r + 16 q (row min(16 t + r, N - 1)) and step s, the 8
    elements k [256 g + 32 s + 8 q, +8) as the 16-byte piece at 1024 s + 16 l,
    zero past K."""
    w = bt.cpu().view(torch.int16).numpy()
    G, tiles = (K + 255) // 256, (N + 15) // 16
    out = np.zeros(tiles * G * 8192, np.uint8)
    for t in range(tiles):
        for g in range(G):
            base = (t * G + g) * 8192
            for lane in range(64):
                n = min(16 * t + lane % 16, N - 1)
                for s in range(8):
                    k0 = 256 * g + 32 * s + 8 * (lane // 16)
                    o = base + 1024 * s + 16 * lane
                    if k0 < K:
                        out[o:o + 16] = w[n, k0:k0 + 8].view(np.uint8)
    return out


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("K", [512, 896])
def test_matmul_pack_layout(dt, K):
    """bi_matmul_pack writes exactly the layout restated in numpy above (20
    rows: the second tile's rows past N repeat row N - 1; two groups, or four
    with the last one zero-filled past K = 896; a row stride past K)."""
    from mlx_batch_invariant_amd import _lib
    N = 20
    wide = randn((N, K + 64), DT[dt], gen(53))
    bt = wide[:, :K]
    lib = _lib.load()
    code = _lib.DTYPE_CODE[DT[dt]]
    nbytes = lib.bi_matmul_pack_bytes(N, K, code)
    got = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")
    _lib.check(lib.bi_matmul_pack(bt.data_ptr(), bt.stride(0), got.data_ptr(), nbytes, N, K, code, None),
               "bi_matmul_pack")
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), _dense_pack_reference(bt, N, K))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_matmul_packed_equals_bi_matmul(dt):
    """bi_matmul_packed with the repacked copy equals bi_matmul bit for bit at
    every M and group count: the streaming GEMV on the copy (16 groups at 131
    column tiles, the last one partial; 8 groups; 32 and 56 groups, A staged or
    read from global memory at 257 and 258 tiles; one partial tile; 4 groups
    with the last one partial, K = 896 (the Qwen2-0.5B linear) and 1000) and
    the row-major launches where the stream does not take the shape (12
    groups; M > 16). The cache behind batch_invariant_matmul(x, W.T) (up to
    PACKED_MAX_M rows) gives the same bits, is found through W's views, goes
    stale on an in-place change of W and is released by drop_packed_weight."""
    from mlx_batch_invariant_amd import _lib
    from mlx_batch_invariant_amd.kernels import matmul as km
    bi = _bi()
    lib = _lib.load()
    code = _lib.DTYPE_CODE[DT[dt]]
    for N, K in ((2048 + 40, 4096), (1000, 2048), (4096 + 8, 14336), (4096 + 24, 8192), (300, 3072), (5, 4096),
                 (4864, 896), (100, 1000)):
        g = gen(N + 7 * K)
        bt = randn((N, K), DT[dt], g)
        x = randn((20, K), DT[dt], g)
        nbytes = lib.bi_matmul_pack_bytes(N, K, code)
        bp = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
        _lib.check(lib.bi_matmul_pack(bt.data_ptr(), bt.stride(0), bp.data_ptr(), nbytes, N, K, code, None),
                   "bi_matmul_pack")
        for M in (1, 3, 5, 8, 12, 16, 20):
            want = _mm(x[:M], bt.t())
            need = lib.bi_matmul_workspace_bytes(M, N, K)
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
            got = torch.empty((M, N), dtype=DT[dt], device="cuda")
            _lib.check(lib.bi_matmul_packed(x.data_ptr(), x.stride(0), bt.data_ptr(), bt.stride(0), bp.data_ptr(),
                                            got.data_ptr(), M, N, K, code, ws.data_ptr(), need, None),
                       "bi_matmul_packed")
            torch.cuda.synchronize()
            assert bits(got) == bits(want), (N, K, M)
    # the cache behind batch_invariant_matmul (last shape's operands)
    W = randn((4096, 4096), DT[dt], gen(59))
    xs = randn((20, 4096), DT[dt], gen(61))
    plain = _mm(xs, W.t())
    bi.cache_packed_weight(W)
    assert km._packed_for(W.t().t()) is not None                # found through a view
    for M in (1, 7, 16, 20):
        assert bits(_mm(xs[:M], W.t())) == bits(plain[:M]), M
    W.add_(0)                                                   # in place: the copy goes stale
    assert km._packed_for(W) is None
    bi.cache_packed_weight(W)
    assert km._packed_for(W) is not None
    bi.drop_packed_weight(W)
    assert km._packed_for(W) is None


def test_linear_packed_under_the_mode():
    """nn.cache_packed_linears on a small model (nn.Linear weights and a
    QuantizedLinear): decode-sized calls under the mode give the same bits with
    and without the repacked copies."""
    bi = _bi()
    from mlx_batch_invariant_amd.kernels import matmul as km
    from mlx_batch_invariant_amd.nn import QuantizedLinear, cache_packed_linears
    torch.manual_seed(0)
    lin = torch.nn.Linear(1024, 512, bias=True).to(torch.bfloat16)
    model = torch.nn.Sequential(torch.nn.Linear(4096, 1024, bias=False), torch.nn.SiLU(), lin).to(
        device="cuda", dtype=torch.bfloat16)
    q = QuantizedLinear.from_linear(torch.nn.Linear(512, 2048, bias=False).to(torch.bfloat16), 64, 4).cuda()
    x = randn((4, 2, 4096), torch.bfloat16, gen(67))
    with torch.no_grad(), bi.set_batch_invariant_mode(strict=True):
        plain = [q(model(x[:, :t])) for t in (1, 2)]
        cache_packed_linears(model)
        cache_packed_linears(q)
        assert km._packed_for(model[0].weight) is not None
        cached = [q(model(x[:, :t])) for t in (1, 2)]
    for p_, c_ in zip(plain, cached):
        assert bits(c_) == bits(p_)
    bi.drop_packed_weight(model[0].weight)
    bi.drop_packed_weight(lin.weight)
    bi.drop_packed(q.weight)
