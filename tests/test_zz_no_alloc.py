"""bi_attn_decode_noalloc (static device scratch instead of a workspace)
against bi_attn_decode with a caller workspace, through the C ABI: bit for bit
on two calls in a row (the second smaller, so stale partials of the first sit
in the shared scratch), and the size limit rejected before launch."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import DT, bits, gen, randn

pytestmark = pytest.mark.gpu


def _lib():
    from mlx_batch_invariant_amd import _lib
    return _lib


def _strides(q3, k, v):
    L = _lib()
    return (L._c_i64 * 8)(q3.stride(0), q3.stride(1), k.stride(0), k.stride(1), k.stride(2),
                          v.stride(0), v.stride(1), v.stride(2))


def _both(B, Hq, Hkv, L, D, dt, lens, seed):
    lib_mod = _lib()
    lib = lib_mod.load()
    g = gen(seed)
    q = randn((B, Hq, D), DT[dt], g)
    k = randn((B, Hkv, L, D), DT[dt], g)
    v = randn((B, Hkv, L, D), DT[dt], g)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    st = _strides(q, k, v)
    sc = D ** -0.5
    code = lib_mod.DTYPE_CODE[DT[dt]]
    stream = lib_mod.stream_of(q)
    out_ws = torch.empty((B, Hq, D), dtype=DT[dt], device="cuda")
    nbytes = lib.bi_attn_decode_workspace_bytes(B, Hq, L, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    lib_mod.check(lib.bi_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kl.data_ptr(), out_ws.data_ptr(),
                                     B, Hq, Hkv, L, D, st, sc, code, ws.data_ptr(), nbytes, stream), "bi_attn_decode")
    out_na = torch.full((B, Hq, D), float("nan"), dtype=DT[dt], device="cuda")
    lib_mod.check(lib.bi_attn_decode_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), kl.data_ptr(),
                                             out_na.data_ptr(), B, Hq, Hkv, L, D, st, sc, code, stream),
                  "bi_attn_decode_noalloc")
    torch.cuda.synchronize()
    return out_ws, out_na


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_noalloc_decode_equals_workspace_decode_twice(dt):
    # first call: many splits and items (dynamic item order, counter in the scratch)
    a_ws, a_na = _both(24, 32, 8, 4100, 128, dt, [4100, 1, 256, 257, 3000] + [1000 + 130 * i for i in range(19)], 1)
    assert bits(a_na) == bits(a_ws)
    # second call, smaller: stale partials and counter of the first call must not leak in
    b_ws, b_na = _both(2, 8, 2, 300, 64, dt, [300, 45], 2)
    assert bits(b_na) == bits(b_ws)


def test_noalloc_decode_rejects_shapes_beyond_the_scratch():
    lib_mod = _lib()
    lib = lib_mod.load()
    assert lib.bi_attn_decode_workspace_bytes(256, 32, 8192, 128) > lib_mod.DECODE_SCRATCH_BYTES
    p = ctypes.c_void_p(256)        # never dereferenced: rejected before any launch
    st = (lib_mod._c_i64 * 8)(*([128] * 8))
    rc = lib.bi_attn_decode_noalloc(p, p, p, None, p, 256, 32, 8, 8192, 128, st, 0.1, lib_mod.BI_BF16, None)
    assert rc == -3, rc
    assert "static scratch" in lib.bi_last_error().decode()


def test_noalloc_decode_captured_in_a_graph_replays_bitwise():
    """One eager call (it resolves the scratch address), then the same call
    captured into a HIP graph: q is refilled between replays, and every replay
    must equal the workspace path on that q, bit for bit."""
    lib_mod = _lib()
    lib = lib_mod.load()
    B, Hq, Hkv, L, D = 4, 32, 8, 1500, 128
    g = gen(7)
    q = randn((B, Hq, D), torch.bfloat16, g)
    k = randn((B, Hkv, L, D), torch.bfloat16, g)
    v = randn((B, Hkv, L, D), torch.bfloat16, g)
    kl = torch.tensor([1500, 3, 700, 256], dtype=torch.int32).cuda()
    st = _strides(q, k, v)
    sc = D ** -0.5
    code = lib_mod.BI_BF16
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device="cuda")
    nbytes = lib.bi_attn_decode_workspace_bytes(B, Hq, L, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")

    def noalloc():
        lib_mod.check(lib.bi_attn_decode_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), kl.data_ptr(),
                                                 out.data_ptr(), B, Hq, Hkv, L, D, st, sc, code,
                                                 lib_mod.stream_of(q)), "bi_attn_decode_noalloc")

    def with_ws():
        ref = torch.empty_like(out)
        lib_mod.check(lib.bi_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kl.data_ptr(), ref.data_ptr(),
                                         B, Hq, Hkv, L, D, st, sc, code, ws.data_ptr(), nbytes,
                                         lib_mod.stream_of(q)), "bi_attn_decode")
        torch.cuda.synchronize()
        return bits(ref)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        noalloc()                      # eager first call on this device's stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert bits(out) == with_ws()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc()
    for seed in (11, 12, 13):
        q.copy_(randn((B, Hq, D), torch.bfloat16, gen(seed)))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = bits(out)
        assert got == with_ws(), f"replay with q seed {seed}"
    del graph

