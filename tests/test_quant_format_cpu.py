"""The torch-side MLX affine format helpers against the oracle (CPU)."""

import numpy as np
import torch

import mlx_batch_invariant_amd as bi
from oracle import bi_oracle as ora


def test_pack_unpack_match_oracle():
    rng = np.random.default_rng(0)
    for bits in (4, 8):
        codes = rng.integers(0, 1 << bits, size=(5, 64))
        w = bi.pack(torch.tensor(codes), bits)
        assert w.dtype == torch.uint32
        assert np.array_equal(w.view(torch.int32).numpy().view(np.uint32), ora.pack(codes, bits))
        assert np.array_equal(bi.unpack(w, bits).numpy(), codes)


def test_quantize_roundtrip_error_and_dequantize_matches_oracle():
    torch.manual_seed(0)
    W = torch.randn(32, 256) * 0.02
    for bits, gs in ((4, 64), (8, 128), (4, 32)):
        wq, s, b = bi.quantize(W, group_size=gs, bits=bits, dtype=torch.bfloat16)
        deq = bi.dequantize(wq, s, b, gs, bits, dtype=torch.bfloat16)
        want = ora.dequantize(wq.view(torch.int32).numpy().view(np.uint32), s.float().numpy(), b.float().numpy(),
                              gs, bits, "bf16")
        assert np.array_equal(deq.float().numpy(), want)
        step = (W.reshape(32, -1, gs).amax(-1) - W.reshape(32, -1, gs).amin(-1)) / ((1 << bits) - 1)
        err = (deq.float() - W).abs().reshape(32, -1, gs).amax(-1)
        assert bool((err <= step * 0.5 + 0.02 * 2 ** -7 * 4).all())
