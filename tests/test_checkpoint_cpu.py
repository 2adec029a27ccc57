"""MLX-affine safetensors checkpoints (mlx_batch_invariant_amd.checkpoint), CPU.

The on-disk layout is MLX's (uint32 words with codes packed low to high,
scales and biases per group, quantization in config.json); the checks pin it
against the oracle's packing and against hand-written safetensors files."""

import json

import numpy as np
import pytest
import torch

import mlx_batch_invariant_amd as bi
from mlx_batch_invariant_amd import checkpoint as ckpt
from mlx_batch_invariant_amd.nn import QuantizedLinear
from oracle import bi_oracle as ora


class Tiny(torch.nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.embed = torch.nn.Embedding(50, 128)
        self.norm = torch.nn.RMSNorm(128, eps=1e-6)
        self.up = torch.nn.Linear(128, 256, bias=False)
        self.down = torch.nn.Linear(256, 128, bias=True)
        self.head = torch.nn.Linear(128, 50, bias=False)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(0.05 * torch.randn(p.shape, generator=g))

    def forward(self, tok):
        h = self.norm(self.embed(tok))
        return self.head(h + self.down(torch.nn.functional.silu(self.up(h))))


def _bits(t):
    return t.detach().contiguous().view(torch.uint8).numpy().tobytes()


def test_save_layout_is_mlx_and_words_match_oracle(tmp_path):
    m = ckpt.quantize_linears(Tiny(), group_size=64, bits=4,
                              predicate=lambda name, lin: name != "head")
    ckpt.save(m, tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["quantization"] == {"group_size": 64, "bits": 4}
    t = ckpt.read_tensors([tmp_path / "model.safetensors"])
    assert t["up.weight"].dtype == torch.uint32 and tuple(t["up.weight"].shape) == (256, 128 * 4 // 32)
    assert tuple(t["up.scales"].shape) == (256, 2) and tuple(t["up.biases"].shape) == (256, 2)
    assert "down.bias" in t and "head.weight" in t and t["head.weight"].dtype == torch.float32
    # packed words: codes low to high, as the oracle packs them
    codes = bi.unpack(t["up.weight"], 4).numpy()
    assert np.array_equal(t["up.weight"].view(torch.int32).numpy().view(np.uint32), ora.pack(codes, 4))
    # dequantized values: the oracle's T(fmaf(code, scale, bias))
    deq = bi.dequantize(t["up.weight"], t["up.scales"], t["up.biases"], 64, 4, dtype=torch.float32)
    want = ora.dequantize(t["up.weight"].view(torch.int32).numpy().view(np.uint32), t["up.scales"].float().numpy(),
                          t["up.biases"].float().numpy(), 64, 4, "f32")
    assert np.array_equal(deq.numpy(), want)


def test_roundtrip_is_bit_exact(tmp_path):
    src = ckpt.quantize_linears(Tiny(), group_size=64, bits=4)
    ckpt.save(src, tmp_path)
    dst = ckpt.load_dir(Tiny(), tmp_path)
    for name in ("up", "down", "head"):
        a, b = src.get_submodule(name), dst.get_submodule(name)
        assert isinstance(b, QuantizedLinear) and (b.group_size, b.bits) == (64, 4)
        for buf in ("weight", "scales", "biases"):
            assert _bits(getattr(a, buf)) == _bits(getattr(b, buf))
    assert _bits(src.down.bias) == _bits(dst.down.bias)
    assert _bits(src.norm.weight) == _bits(dst.norm.weight)
    tok = torch.tensor([[1, 2, 3, 4]])
    assert _bits(src(tok)) == _bits(dst(tok))


def test_per_layer_quantization_and_shards(tmp_path):
    m = Tiny()
    ckpt.quantize_linears(m, group_size=64, bits=4, predicate=lambda n, l: n == "up")
    ckpt.quantize_linears(m, group_size=128, bits=8, predicate=lambda n, l: n == "down")
    ckpt.save(m, tmp_path, shard_bytes=20_000)
    shards = sorted(tmp_path.glob("*.safetensors"))
    assert len(shards) > 1 and all("-of-" in s.name for s in shards)
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["quantization"]["down"] == {"group_size": 128, "bits": 8}
    assert ckpt.quantization_for(cfg, "up") == {"group_size": 64, "bits": 4}
    out = ckpt.load_dir(Tiny(), tmp_path)
    assert (out.up.bits, out.up.group_size, out.down.bits, out.down.group_size) == (4, 64, 8, 128)
    assert isinstance(out.head, torch.nn.Linear)
    assert _bits(out.down.weight) == _bits(m.down.weight)


def test_hand_written_mlx_file_loads(tmp_path):
    """A file written the way MLX writes it (not by this module): words from
    the oracle's packer, fp16 scales/biases, config.json with the defaults."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(1)
    N, K, gs, bits = 8, 128, 64, 4
    codes = rng.integers(0, 16, size=(N, K))
    words = torch.from_numpy(ora.pack(codes, bits).view(np.int32)).view(torch.uint32)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, size=(N, K // gs)).astype(np.float16))
    biases = torch.from_numpy(rng.uniform(-0.05, 0.05, size=(N, K // gs)).astype(np.float16))
    save_file({"proj.weight": words, "proj.scales": scales, "proj.biases": biases}, str(tmp_path / "model.safetensors"),
              metadata={"format": "mlx"})
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"group_size": gs, "bits": bits}}))
    m = torch.nn.Module()
    m.proj = torch.nn.Linear(K, N, bias=False)
    ckpt.load_dir(m, tmp_path)
    assert isinstance(m.proj, QuantizedLinear)
    assert np.array_equal(bi.unpack(m.proj.weight.view(torch.uint32), bits).numpy(), codes)
    x = torch.randn(3, K, dtype=torch.float16)
    W = ora.dequantize(ora.pack(codes, bits), scales.float().numpy(), biases.float().numpy(), gs, bits, "f16")
    ref = torch.matmul(x.float(), torch.from_numpy(W).float().t())
    assert torch.allclose(m.proj(x).float(), ref, rtol=1e-2, atol=1e-3)


def test_strict_mismatch_raises(tmp_path):
    ckpt.save(ckpt.quantize_linears(Tiny()), tmp_path)
    t = ckpt.read_tensors(sorted(tmp_path.glob("*.safetensors")))
    t.pop("norm.weight")
    with pytest.raises(KeyError):
        ckpt.load_into(Tiny(), t, {"quantization": {"group_size": 64, "bits": 4}})
    t2 = ckpt.read_tensors(sorted(tmp_path.glob("*.safetensors")))
    t2["extra.weight"] = torch.zeros(1)
    with pytest.raises(KeyError):
        ckpt.load_into(Tiny(), t2, {"quantization": {"group_size": 64, "bits": 4}})
    bad = dict(ckpt.read_tensors(sorted(tmp_path.glob("*.safetensors"))))
    bad["up.scales"] = bad["up.scales"][:, :1]
    with pytest.raises(ValueError):
        ckpt.load_into(Tiny(), bad, {"quantization": {"group_size": 64, "bits": 4}})
