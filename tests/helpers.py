"""Shared test helpers: tensor <-> numpy, bit comparison, seeded inputs."""

from __future__ import annotations

import math

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


def gpu_exp2(x) -> np.ndarray:
    """The attention kernels' hardware exp2 (bi_exp2_f32, v_exp_f32) of a
    float32 array, evaluated on the GPU: the exp2 argument of the oracle's
    matrix-core emulation in the GPU tests."""
    from mlx_batch_invariant_amd import _lib
    x = np.ascontiguousarray(x, np.float32)
    if x.size == 0:
        return x.copy()
    xs = torch.from_numpy(x.reshape(-1)).cuda()
    y = torch.empty_like(xs)
    _lib.check(_lib.load().bi_exp2_f32(xs.data_ptr(), y.data_ptr(), xs.numel(), _lib.stream_of(xs)), "bi_exp2_f32")
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(x.shape)


def attn_bound(q, k, v, scale, causal, dtype, kv_lens=None) -> np.ndarray:
    """Per-element bound on how far the matrix-core order and the reference's
    per-key order of the same attention may differ before the final rounding
    (both start from the same bf16 / f16 / f32 inputs). With
    A = sum_j p_j |v_j| / sum_j p_j (float64 closed form on |v|) per output,
    the bound is 2 A (e_p + e_acc + 2 e_s):
      e_p   = 2^-17 (bf16) / 2^-21 (f16) / 0 (f32): the matrix-core kernels
              carry a 16-bit weight p as hi + lo (8 + 8 or 11 + 11 bits);
      e_acc = (2 * 256 + 2 * nsplit) 2^-24: the per-key order rescales its
              running sums once per key of a split (corr) and once per split,
              the matrix-core order rounds once per MFMA block and merge;
      e_s   = ln 2 (D + 2) 2^-24 S: a score's fp32 error over D products,
              S = the row's largest sum_d |q_d k_d| scale log2(e); a weight's
              argument s - m carries two such errors;
    the factor 2 covers the normalisation by the same perturbed weights."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    from oracle import bi_oracle as ora
    B, Hq, Tq, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    A = ora.attention_float64(q, k, np.abs(v), scale, causal, kv_lens=kv_lens)
    e_p = {"bf16": 2.0 ** -17, "f16": 2.0 ** -21, "f32": 0.0}[dtype]
    S = np.zeros((B, Hq, Tq))
    ns = np.zeros((B,))
    for b in range(B):
        n = L if kv_lens is None else min(max(int(kv_lens[b]), 0), L)
        ns[b] = -(-n // 256)
        if n == 0:
            continue
        for h in range(Hq):
            S[b, h] = (np.abs(q[b, h]) @ np.abs(k[b, h // G, :n]).T).max(-1) * abs(scale) * 1.4426950408889634
    e_acc = (2 * 256 + 2 * ns)[:, None, None] * 2.0 ** -24
    e_s = math.log(2) * (D + 2) * 2.0 ** -24 * S
    return 2 * A * (e_p + e_acc + 2 * e_s)[..., None]


def attn_bound_check(got, want, q, k, v, scale, causal, dtype, kv_lens=None) -> float:
    """|got - want| <= half a storage ulp of each + attn_bound, element by
    element; returns the worst ratio of the difference to that allowance."""
    from oracle import bi_oracle as ora
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    # both sides are rounded to the storage type: half an ulp each, plus the bound
    allow = 0.5 * (ora.ulp(want, dtype) + ora.ulp(got, dtype)) + attn_bound(q, k, v, scale, causal, dtype, kv_lens)
    ratio = np.abs(got - want) / allow
    worst = float(ratio.max()) if ratio.size else 0.0
    assert worst <= 1.0, f"attention order difference {worst:.3f} x the stated bound; " + ora.isclose_report(got, want)
    return worst
