"""Hardware known-answer vectors of one gfx950 matrix-core step, taken through
the single-instruction probe bi_mfma_step_probe (no matmul kernel involved).

    python tests/golden/make_mfma_step_golden.py      # on an MI355X, after the build

Each block is one step d = c + A B^T with caller-chosen operands and a live
fp32 accumulator c: one v_mfma_f32_16x16x32_{bf16,f16}, or for fp32 the
kernels' eight v_mfma_f32_16x16x4_f32. The operands are regenerated from the
seed by ``step_operands`` (numpy's PCG64 stream), so the file holds only the
outputs d. The CPU suite checks the oracle's ``mfma_step`` against this file
bit for bit; the GPU suite checks that the file still reproduces on the GPU
it runs on, and the model on fresh operands.

Operand kinds (a, b: [blocks, 16, 32] in k-slot order; c: [blocks, 16, 16]):
  normal  N(0, 1) operands, accumulator N(0, 4);
  wide    operands and accumulator spread over 2^-8 .. 2^8 (products many
          binades apart);
  accbig  accumulator 2^10 .. 2^16 above the products (the products enter
          through the low end of the accumulator's window);
  cancel  accumulator close to minus the exact step sum (massive
          cancellation; the result exposes the block-wise truncation);
  sparse  one nonzero product per lane quarter, the rest exact zeros, and
          whole quarters of zeros (a block with no product leaves the
          accumulator unchanged);
  tiny    16-bit operands at the bottom of their range, subnormals included
          (the multiplier's exponent of a subnormal operand is the type's
          minimum normal exponent).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "mfma_step_gfx950.npz"
FIXTURE_SEED = 9
KINDS = ("normal", "wide", "accbig", "cancel", "sparse", "tiny")
DTYPES = ("bf16", "f16", "f32")
BLOCKS = 24


def _round(x: np.ndarray, dt: str) -> np.ndarray:
    import torch
    t = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(t).float().numpy()


def _sig(rng, shape, bits, emin, emax):
    """Random signs, `bits`-bit significands and exponents in [emin, emax]."""
    s = rng.choice([-1.0, 1.0], size=shape)
    m = 1 + rng.integers(0, 1 << (bits - 1), size=shape) / float(1 << (bits - 1))
    return s * m * np.exp2(rng.integers(emin, emax + 1, size=shape))


def step_operands(dt: str, kind: str, seed: int, blocks: int = BLOCKS):
    """(a [blocks, 16, 32], b [blocks, 16, 32], c [blocks, 16, 16]) float32
    values: a and b hold values of type ``dt``, c any fp32."""
    rng = np.random.default_rng([seed, KINDS.index(kind), DTYPES.index(dt)])
    shp, cshp = (blocks, 16, 32), (blocks, 16, 16)
    sb = 8 if dt == "bf16" else 11 if dt == "f16" else 24
    e16 = 5 if dt == "f16" else 8                       # keep f16 products inside its range
    if kind == "normal":
        a, b = rng.standard_normal(shp), rng.standard_normal(shp)
        c = 2 * rng.standard_normal(cshp)
    elif kind == "wide":
        a, b = _sig(rng, shp, sb, -e16, e16), _sig(rng, shp, sb, -e16, e16)
        c = _sig(rng, cshp, 24, -2 * e16, 2 * e16)
    elif kind == "accbig":
        a, b = _sig(rng, shp, sb, -4, 4), _sig(rng, shp, sb, -4, 4)
        c = _sig(rng, cshp, 24, 10, 16)
    elif kind == "cancel":
        a, b = _sig(rng, shp, sb, -6, 6), _sig(rng, shp, sb, -6, 6)
        a, b = _round(a, dt), _round(b, dt)
        exact = np.einsum("zik,zjk->zij", a.astype(np.float64), b.astype(np.float64))
        c = -exact * (1 + _sig(rng, cshp, 6, -30, -20))          # within 2^-20 of the negated sum
    elif kind == "sparse":
        a, b = _sig(rng, shp, sb, -6, 6), _sig(rng, shp, sb, -6, 6)
        keep = np.zeros(shp, bool)
        lead = rng.integers(0, 8, size=(blocks, 16, 4))
        for q in range(4):
            np.put_along_axis(keep[..., 8 * q:8 * q + 8], lead[..., q:q + 1], True, axis=-1)
        keep &= rng.random((blocks, 16, 1)) < 0.85                  # some rows: every quarter empty
        a = np.where(keep, a, 0.0)
        c = _sig(rng, cshp, 24, -8, 8)
    else:  # tiny
        lo = {"bf16": -133, "f16": -24, "f32": -60}[dt]
        hi = {"bf16": -118, "f16": -10, "f32": -40}[dt]
        a = _sig(rng, shp, sb, lo, hi)
        b = _sig(rng, shp, sb, 0, 2 if dt != "f16" else 1)
        c = _sig(rng, cshp, 24, hi - 2, hi + 6) if dt != "f16" else _sig(rng, cshp, 24, -20, -6)
    return _round(a, dt), _round(b, dt), np.asarray(c, np.float32)


def probe(a, b, c, dt: str) -> np.ndarray:
    """d [blocks, 16, 16] of the hardware step on (a, b, c), through the C ABI."""
    import torch
    from mlx_batch_invariant_amd import _lib
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    ad = torch.from_numpy(np.ascontiguousarray(a)).to(tdt).cuda()
    bd = torch.from_numpy(np.ascontiguousarray(b)).to(tdt).cuda()
    cd = torch.from_numpy(np.ascontiguousarray(c, np.float32)).cuda()
    dd = torch.empty_like(cd)
    rc = _lib.load().bi_mfma_step_probe(ad.data_ptr(), bd.data_ptr(), cd.data_ptr(), dd.data_ptr(), a.shape[0],
                                        _lib.DTYPE_CODE[tdt], _lib.stream_of(cd))
    _lib.check(rc, "bi_mfma_step_probe")
    torch.cuda.synchronize()
    return dd.cpu().numpy()


def model(a, b, c, dt: str) -> np.ndarray:
    """The oracle's step on the same operands: d[z, i, j] = mfma_step(c[z, i, j], a[z, i], b[z, j])."""
    from oracle import bi_oracle as ora
    return ora.mfma_step(c, a[:, :, None, :], b[:, None, :, :], dt)


def main() -> int:
    root = HERE.parent.parent
    sys.path[:0] = [str(root), str(root / "mlx-batch-invariant_amd")]
    out = {}
    for dt in DTYPES:
        for kind in KINDS:
            a, b, c = step_operands(dt, kind, FIXTURE_SEED)
            d = probe(a, b, c, dt)
            out[f"{dt}_{kind}"] = d
            same = float(np.mean(d.view(np.uint32) == model(a, b, c, dt).view(np.uint32)))
            print(dt, kind, "model agreement", same, flush=True)
    dest = Path(sys.argv[1]) if len(sys.argv) > 1 else FIXTURE
    np.savez_compressed(dest, **out)
    print("wrote", dest)
    return 0


if __name__ == "__main__":
    sys.exit(main())
