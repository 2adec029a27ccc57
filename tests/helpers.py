"""Shared test helpers: tensor <-> numpy, bit comparison, seeded inputs."""

from __future__ import annotations

import numpy as np
import torch

DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def bits(t: torch.Tensor) -> bytes:
    """Raw bytes of a tensor (bf16 compared bitwise too)."""
    t = t.detach().contiguous()
    return t.view(torch.uint8).cpu().numpy().tobytes() if t.dtype != torch.bool else t.cpu().numpy().tobytes()


def randn(shape, dtype, gen, scale=1.0, device="cuda"):
    return (torch.randn(shape, generator=gen) * scale).to(dtype).to(device)


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def assert_bits_equal(got, want, what: str = "") -> None:
    """Bitwise equality of two float32 arrays (values of any storage type),
    with a report of how many elements differ and by how much."""
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    diff = got.view(np.uint32) != want.view(np.uint32)
    if diff.any():
        i = int(np.argmax(diff))
        raise AssertionError(f"{what}: {int(diff.sum())} of {diff.size} elements differ; first at flat {i}: "
                             f"got {got.flat[i]!r} want {want.flat[i]!r}; "
                             f"max |diff| {float(np.abs(got.astype(np.float64) - want)[diff].max()):.3e}")
