"""Hardware known-answer vectors of the gfx950 matrix-core accumulation.

    python tests/golden/make_mfma_golden.py      # on an MI355X, after the build

Runs bi_matmul's split launch (M <= 32 rows, more than 64 K groups: every
group's raw fp32 partial, 8 MFMA steps from zero, lands in the caller's
workspace) on seeded operands and stores a sample of the partials in
tests/golden/mfma_gfx950.npz. The operands are regenerated from the seed by
``operands`` (numpy's PCG64 stream), so the file holds only outputs. The CPU
suite checks the oracle's MFMA model against this file bit for bit; the GPU
suite checks that the file still reproduces on the GPU it runs on.

Operand kinds:
  normal   N(0, 1) values rounded to the type (scale of real activations);
  wide     N(0, 1) times 2^U{-8..8} (products many binades apart: heavy
           truncation and cancellation inside an MFMA block);
  crafted  8-bit significands with random exponents, with the K groups
           cycling through four patterns of live steps (only step 0: one MFMA
           from zero; steps 0-1: an MFMA into a live accumulator; all eight;
           step 0 at twice the exponent range).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "mfma_gfx950.npz"
FIXTURE_SEED = 5
KINDS = ("normal", "wide", "crafted")
M, N, G = 16, 64, 65          # 65 groups of 256: the split launch for M <= 16
SAMPLE_GROUPS, SAMPLE_COLS = 4, 16


def _round(x: np.ndarray, dt: str) -> np.ndarray:
    import torch
    t = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(t).float().numpy()


def _sig8(rng, shape, emin, emax):
    s = rng.choice([-1.0, 1.0], size=shape)
    return s * (1 + rng.integers(0, 128, size=shape) / 128.0) * np.exp2(rng.integers(emin, emax + 1, size=shape))


def operands(dt: str, kind: str, seed: int):
    """a [M, G*256], bt [N, G*256] float32 holding values of type ``dt``."""
    rng = np.random.default_rng([seed, KINDS.index(kind), ("bf16", "f16", "f32").index(dt)])
    K = G * 256
    if kind == "normal":
        a, b = rng.standard_normal((M, K)), rng.standard_normal((N, K))
    elif kind == "wide":
        a = rng.standard_normal((M, K)) * np.exp2(rng.integers(-8, 9, (M, K)))
        b = rng.standard_normal((N, K)) * np.exp2(rng.integers(-8, 9, (N, K)))
        if dt == "f16":
            a, b = a / 64, b / 64               # keep f16 products inside its range
    else:
        e = 5 if dt == "f16" else 6
        a, b = _sig8(rng, (M, K), -e, e), _sig8(rng, (N, K), -e, e)
        for g in range(G):
            base, pat = 256 * g, g % 4
            if pat in (0, 3):
                a[:, base + 32:base + 256] = 0
            if pat == 1:
                a[:, base + 64:base + 256] = 0
            if pat == 3:
                a[:, base:base + 32] = _sig8(rng, (M, 32), -2 * e, 2 * e) if dt != "f16" else _sig8(rng, (M, 32), -7, 7)
    return _round(a, dt), _round(b, dt)


def split_partials(a_dev, bt_dev):
    """(out, partials [G, M, N] fp32 numpy) of one split launch, through the C ABI."""
    import torch
    from mlx_batch_invariant_amd import _lib
    lib = _lib.load()
    m, k = a_dev.shape
    n = bt_dev.shape[0]
    nbytes = lib.bi_matmul_workspace_bytes(m, n, k)
    g = nbytes // (4 * m * n)
    assert nbytes > 0 and g == -(-k // 256), "the shape must take the split launch"
    ws = torch.zeros(nbytes // 4, dtype=torch.float32, device=a_dev.device)
    out = torch.empty((m, n), dtype=a_dev.dtype, device=a_dev.device)
    rc = lib.bi_matmul(a_dev.data_ptr(), a_dev.stride(0), bt_dev.data_ptr(), bt_dev.stride(0), out.data_ptr(), m, n,
                       k, _lib.DTYPE_CODE[a_dev.dtype], ws.data_ptr(), nbytes, _lib.stream_of(a_dev))
    _lib.check(rc, "bi_matmul")
    torch.cuda.synchronize()
    return out, ws.reshape(g, m, n).cpu().numpy()


def sample(part: np.ndarray) -> np.ndarray:
    """The stored part of a [G, M, N] partial array: the first SAMPLE_GROUPS
    groups (one of each crafted pattern) and SAMPLE_COLS columns."""
    return np.ascontiguousarray(part[:SAMPLE_GROUPS, :, :SAMPLE_COLS])


def main() -> int:
    root = HERE.parent.parent
    sys.path[:0] = [str(root), str(root / "mlx-batch-invariant_amd")]
    import torch
    dts = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    out = {}
    for dt, tdt in dts.items():
        for kind in KINDS:
            a, bt = operands(dt, kind, FIXTURE_SEED)
            _, part = split_partials(torch.from_numpy(a).to(tdt).cuda(), torch.from_numpy(bt).to(tdt).cuda())
            out[f"{dt}_{kind}"] = sample(part)
            print(dt, kind, "ok", flush=True)
    dest = Path(sys.argv[1]) if len(sys.argv) > 1 else FIXTURE
    np.savez_compressed(dest, **out)
    print("wrote", dest)
    return 0


if __name__ == "__main__":
    sys.exit(main())
