"""torch.ops.mlx_bi.* on the GPU: same bits as the Python functions, opcheck,
and a torch.compile graph (aot_eager backend: no generated kernels) that keeps
the ops."""

import pytest
import torch

from helpers import bits, gen, randn

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _inputs():
    g = gen(0)
    bi = _bi()
    a = randn((6, 256), torch.bfloat16, g)
    w = randn((256, 96), torch.bfloat16, g, scale=0.05)
    W = torch.randn((128, 256), generator=g) * 0.02
    wq, s, b = bi.quantize(W, group_size=64, bits=4, dtype=torch.bfloat16)
    gam = (1 + 0.1 * torch.randn(256, generator=g)).to(torch.bfloat16).cuda()
    bet = (0.1 * torch.randn(256, generator=g)).to(torch.bfloat16).cuda()
    q = randn((2, 8, 5, 64), torch.bfloat16, g)
    k = randn((2, 2, 40, 64), torch.bfloat16, g)
    v = randn((2, 2, 40, 64), torch.bfloat16, g)
    return a, w, (wq.view(torch.int32).cuda(), s.cuda(), b.cuda()), gam, bet, (q, k, v)


def test_ops_equal_python_functions():
    bi = _bi()
    a, w, (wq, s, b), gam, bet, (q, k, v) = _inputs()
    ops = torch.ops.mlx_bi
    assert bits(ops.matmul(a, w)) == bits(bi.batch_invariant_matmul(a, w))
    a3 = a.reshape(2, 3, 256)
    w3 = torch.stack([w, w.flip(0)])
    assert bits(ops.matmul(a3, w3)) == bits(bi.batch_invariant_bmm(a3, w3))
    assert bits(ops.quantized_matmul(a, wq, s, b, 64, 4)) == bits(
        bi.batch_invariant_quantized_matmul(a, wq, s, b, group_size=64, bits=4))
    assert bits(ops.rms_norm(a, gam, 1e-6)) == bits(bi.batch_invariant_rms_norm(a, gam, 1e-6))
    assert bits(ops.layer_norm(a, gam, bet, 1e-5)) == bits(bi.batch_invariant_layer_norm(a, gam, bet, 1e-5))
    assert bits(ops.attention(q, k, v, 0.125, True, None)) == bits(
        bi.batch_invariant_attention(q, k, v, scale=0.125, mask="causal"))
    assert bits(ops.attention(q[:, :, :1], k, v, 0.125, False, None)) == bits(
        bi.batch_invariant_attention(q[:, :, :1], k, v, scale=0.125))
    # a one-page-per-64-keys pool holding the same keys in order
    kp = torch.zeros((2, 2, 64, 64), dtype=k.dtype, device=k.device)
    vp = torch.zeros_like(kp)
    kp[:, :, :40] = k
    vp[:, :, :40] = v
    table = torch.arange(2, dtype=torch.int32, device=k.device).reshape(2, 1)
    lens = torch.full((2,), 40, dtype=torch.int32, device=k.device)
    assert bits(ops.paged_attention(q, kp, vp, table, lens, 0.125, True)) == bits(
        bi.batch_invariant_attention(q, k, v, scale=0.125, mask="causal"))


def test_opcheck():
    a, w, (wq, s, b), gam, bet, (q, k, v) = _inputs()
    ops = torch.ops.mlx_bi
    tests = ("test_schema", "test_faketensor")
    torch.library.opcheck(ops.matmul.default, (a, w), test_utils=tests)
    torch.library.opcheck(ops.quantized_matmul.default, (a, wq, s, b, 64, 4), test_utils=tests)
    torch.library.opcheck(ops.rms_norm.default, (a, gam, 1e-6), test_utils=tests)
    torch.library.opcheck(ops.layer_norm.default, (a, gam, bet, 1e-5), test_utils=tests)
    torch.library.opcheck(ops.attention.default, (q, k, v, 0.125, True, None), test_utils=tests)


def test_compiled_graph_keeps_the_kernels():
    a, w, _, gam, bet, _ = _inputs()

    def block(x):
        h = torch.ops.mlx_bi.layer_norm(x, gam, bet, 1e-5)
        return torch.ops.mlx_bi.matmul(torch.nn.functional.silu(h), w)

    eager = block(a)
    compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    for m in (6, 6, 3):                     # the rows of a smaller batch: same bits
        assert bits(compiled(a[:m])) == bits(eager[:m])
