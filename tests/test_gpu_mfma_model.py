"""Probe of the MFMA accumulation model through the split launch's fp32 group
partials (the analogue of the reference's hardware-layout known-answer test,
tests/test_batch_invariance.py:135-149).

For M <= 32 and more than 64 K groups, bi_matmul writes every group partial
acc_g (fp32, before the fold) to the caller's workspace. Reading it back shows
the MFMA chain's own rounding at fp32 precision, which the bf16 outputs hide.
The test checks the partials against the oracle's model (each 32-wide step
adds the exact sum of its products to the accumulator with one fp32 rounding)
within an fp32 bound, records how often they agree bit for bit, and checks
that the fold kernel's output is exactly the oracle fold of the GPU partials.
"""

import json
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import gen, randn, to_np
from oracle import bi_oracle as ora

pytestmark = pytest.mark.gpu

OUT = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"


def _split_partials(a, bt):
    from mlx_batch_invariant_amd import _lib
    lib = _lib.load()
    M, K = a.shape
    N = bt.shape[0]
    nbytes = lib.bi_matmul_workspace_bytes(M, N, K)
    assert nbytes > 0
    ws = torch.zeros(nbytes // 4, dtype=torch.float32, device="cuda")
    out = torch.empty((M, N), dtype=a.dtype, device="cuda")
    rc = lib.bi_matmul(a.data_ptr(), a.stride(0), bt.data_ptr(), bt.stride(0), out.data_ptr(), M, N, K,
                       _lib.DTYPE_CODE[a.dtype], ws.data_ptr(), nbytes, _lib.stream_of(a))
    _lib.check(rc, "bi_matmul")
    torch.cuda.synchronize()
    G = nbytes // (4 * M * N)
    return out, ws.reshape(G, M, N)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_split_partials_follow_the_mfma_model(dt):
    M, N, K = 16, 64, 65 * 256           # > 64 groups: the split launch
    g = gen(21)
    a = randn((M, K), torch.bfloat16 if dt == "bf16" else torch.float16, g)
    bt = randn((N, K), a.dtype, g)
    out, part = _split_partials(a, bt)
    got = part.cpu().numpy()
    want = ora.group_partials(to_np(a), to_np(bt), dt)
    exact = float(np.mean(got == want))
    # bound: 2 fp32 roundings' worth of the step sums' magnitude, per group
    a64, b64 = np.abs(to_np(a).astype(np.float64)), np.abs(to_np(bt).astype(np.float64))
    G = K // 256
    bound = np.stack([a64[:, 256 * i:256 * i + 256] @ b64[:, 256 * i:256 * i + 256].T for i in range(G)]) * 2 ** -21
    assert np.all(np.abs(got - want) <= bound)
    # the fold kernel is exactly the oracle's fold of these partials
    total = np.zeros((M, N), np.float32)
    for i in range(G):
        total = (total + got[i]).astype(np.float32)
    assert np.array_equal(to_np(out), ora.round_to(total, dt))
    report = {"dtype": dt, "exact_fraction_vs_single_rounding_step_model": exact,
              "max_abs_diff": float(np.abs(got - want).max())}
    if OUT.is_dir():
        (OUT / f"mfma_model_{dt}.json").write_text(json.dumps(report, indent=1))
    print(report)
