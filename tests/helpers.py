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
