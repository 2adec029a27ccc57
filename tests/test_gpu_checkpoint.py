"""An MLX-affine checkpoint through the kernels (the integration path): a model
quantized and saved in MLX's on-disk layout (reference format:
kernels/quantized.py:1-8), loaded back into QuantizedLinear layers and run on
the GPU under the mode equals the oracle's dequantize + matmul bit for bit, per
layer, for the 4-bit and 8-bit layers, with and without bias, and for the dense
layer left unquantized."""

import numpy as np
import pytest
import torch

from helpers import assert_bits_equal, gen, to_np
from oracle import bi_oracle as ora

pytestmark = pytest.mark.gpu


class Net(torch.nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.norm = torch.nn.RMSNorm(512, eps=1e-6)
        self.up = torch.nn.Linear(512, 1024, bias=False)
        self.down = torch.nn.Linear(1024, 512, bias=True)
        self.head = torch.nn.Linear(512, 320, bias=False)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(0.05 * torch.randn(p.shape, generator=g))


def _words(t):
    return t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32)


def test_loaded_checkpoint_layers_equal_the_oracle(tmp_path):
    import mlx_batch_invariant_amd as bi
    from mlx_batch_invariant_amd import checkpoint as ckpt
    src = Net().to(torch.bfloat16)
    ckpt.quantize_linears(src, group_size=64, bits=4, predicate=lambda n, l: n == "up")
    ckpt.quantize_linears(src, group_size=128, bits=8, predicate=lambda n, l: n == "down")
    ckpt.save(src, tmp_path)
    m = ckpt.load_dir(Net().to(torch.bfloat16), tmp_path).cuda()
    assert (m.up.bits, m.up.group_size, m.down.bits, m.down.group_size) == (4, 64, 8, 128)
    assert isinstance(m.head, torch.nn.Linear)

    x = (torch.randn((24, 512), generator=gen(3)) * 0.5).to(torch.bfloat16).cuda()
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True), torch.no_grad():
        h = m.norm(x)
        u = m.up(h)
        a = torch.nn.functional.silu(u)
        d = m.down(a)
        y = m.head(h + d)
    st = bi.stats()["handled"]
    assert st.get("quantized_matmul", 0) >= 2 and st.get("rms_norm", 0) >= 1

    # RMSNorm (weight from the checkpoint)
    assert_bits_equal(to_np(h), ora.rms_norm(to_np(x), to_np(m.norm.weight), 1e-6, "bf16"), "norm")
    # 4-bit g64 layer: oracle dequantize of the loaded words, then the quantized k-slot order
    Wu = ora.dequantize(_words(m.up.weight), to_np(m.up.scales), to_np(m.up.biases), 64, 4, "bf16")
    assert_bits_equal(to_np(u), ora.matmul(to_np(h), Wu, "bf16", kmap="blocked"), "up (4-bit g64)")
    # 8-bit g128 layer with bias: the matmul, then torch's bf16 add of the bias
    Wd = ora.dequantize(_words(m.down.weight), to_np(m.down.scales), to_np(m.down.biases), 128, 8, "bf16")
    mm = ora.matmul(to_np(a), Wd, "bf16", kmap="blocked")
    assert_bits_equal(to_np(d), ora.round_to(mm + to_np(m.down.bias)[None, :], "bf16"), "down (8-bit g128 + bias)")
    # dense layer
    assert_bits_equal(to_np(y), ora.matmul(to_np(h + d), to_np(m.head.weight), "bf16"), "head (dense)")
    # the on-disk words are the ones that were saved
    assert np.array_equal(_words(m.up.weight), _words(src.up.weight))
