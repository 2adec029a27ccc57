"""torch.ops.mlx_bi.* registration (CPU): schemas, fake-tensor shape rules,
and the loud failure for tensors that are not on the GPU."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import mlx_batch_invariant_amd  # noqa: F401  (registers the ops)

OPS = ["matmul", "quantized_matmul", "rms_norm", "layer_norm", "attention", "paged_attention"]


def test_ops_are_registered_with_schemas():
    for name in OPS:
        op = getattr(torch.ops.mlx_bi, name)
        assert str(op.default._schema).startswith(f"mlx_bi::{name}(")


def test_fake_shapes_and_dtypes():
    with FakeTensorMode():
        a = torch.empty(5, 7, 64, dtype=torch.bfloat16)
        w = torch.empty(64, 30, dtype=torch.bfloat16)
        assert torch.ops.mlx_bi.matmul(a, w).shape == (5, 7, 30)
        b3 = torch.empty(3, 1, 64, 9, dtype=torch.float32)
        out = torch.ops.mlx_bi.matmul(a, b3)
        assert out.shape == (3, 5, 7, 9) and out.dtype == torch.float32
        wq = torch.empty(100, 64 * 4 // 32, dtype=torch.int32)
        s = torch.empty(100, 1, dtype=torch.bfloat16)
        assert torch.ops.mlx_bi.quantized_matmul(a, wq, s, s, 64, 4).shape == (5, 7, 100)
        assert torch.ops.mlx_bi.rms_norm(a, None, 1e-6).shape == a.shape
        assert torch.ops.mlx_bi.layer_norm(a, None, None, 1e-5).shape == a.shape
        q = torch.empty(2, 8, 3, 64, dtype=torch.bfloat16)
        kv = torch.empty(2, 2, 40, 64, dtype=torch.bfloat16)
        assert torch.ops.mlx_bi.attention(q, kv, kv, 0.125, True, None).shape == q.shape
        pool = torch.empty(9, 2, 16, 64, dtype=torch.bfloat16)
        table = torch.empty(2, 3, dtype=torch.int32)
        assert torch.ops.mlx_bi.paged_attention(q, pool, pool, table, None, 0.125, True).shape == q.shape


def test_cpu_tensors_fail_loudly():
    x = torch.randn(3, 64)
    with pytest.raises(ValueError, match="GPU"):
        torch.ops.mlx_bi.rms_norm(x, None, 1e-6)
    with pytest.raises(ValueError, match="GPU"):
        torch.ops.mlx_bi.matmul(x, torch.randn(64, 5))
