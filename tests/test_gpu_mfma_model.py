"""The oracle's model of the gfx950 matrix-core accumulation against the
hardware, through the split launch's fp32 group partials (the analogue of the
reference's hardware-layout known-answer test,
tests/test_batch_invariance.py:135-149).

For M <= 32 and more than 64 K groups, bi_matmul writes every group partial
acc_g (fp32, 8 MFMA steps from zero, before the fold) to the caller's
workspace. Reading it back shows the MFMA chain's own rounding at fp32
precision, which the bf16 outputs hide. The partials must equal the oracle's
``group_partials`` bit for bit on realistic, wide-range and crafted
operands, and the fold kernel's output must be the oracle fold of them.
"""

import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, to_np
from oracle import bi_oracle as ora

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_mfma_golden as mg  # noqa: E402

pytestmark = pytest.mark.gpu

OUT = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("kind", mg.KINDS)
def test_split_partials_equal_the_mfma_model(dt, kind):
    a, bt = mg.operands(dt, kind, seed=31)
    out, part = mg.split_partials(torch.from_numpy(a).to(DT[dt]).cuda(), torch.from_numpy(bt).to(DT[dt]).cuda())
    want = ora.group_partials(a, bt, dt)
    exact = float(np.mean(part.view(np.uint32) == want.view(np.uint32)))
    if OUT.is_dir():
        (OUT / f"mfma_model_{dt}_{kind}.json").write_text(json.dumps({"dtype": dt, "kind": kind, "exact": exact}))
    assert_bits_equal(part, want, f"{dt} {kind}")
    total = np.zeros(part.shape[1:], np.float32)
    for g in range(part.shape[0]):
        total = (total + part[g]).astype(np.float32)
    assert_bits_equal(to_np(out), ora.round_to(total, dt), "fold")


def test_committed_fixture_reproduces_on_this_gpu():
    """The hardware vectors in tests/golden/mfma_gfx950.npz come back bit for
    bit from this GPU (the CPU suite checks the oracle against the same file)."""
    fx = np.load(mg.FIXTURE)
    for dt in ("bf16", "f16", "f32"):
        for kind in mg.KINDS:
            a, bt = mg.operands(dt, kind, seed=mg.FIXTURE_SEED)
            _, part = mg.split_partials(torch.from_numpy(a).to(DT[dt]).cuda(), torch.from_numpy(bt).to(DT[dt]).cuda())
            assert_bits_equal(mg.sample(part), fx[f"{dt}_{kind}"], f"{dt} {kind}")


# ---------------------------------------------------------------------------
# One matrix-core step on its own (bi_mfma_step_probe): the same model,
# pinned through the instruction alone, with live accumulators.
# ---------------------------------------------------------------------------
import make_mfma_step_golden as sg  # noqa: E402


@pytest.mark.parametrize("dt", sg.DTYPES)
@pytest.mark.parametrize("kind", sg.KINDS)
def test_single_step_equals_the_mfma_model(dt, kind):
    """d = c + A B^T by the instruction (no matmul kernel involved) equals the
    oracle's mfma_step bit for bit on fresh operands of every kind: large and
    cancelling accumulators, sparse and empty quarters, subnormal operands."""
    a, b, c = sg.step_operands(dt, kind, seed=77, blocks=64)
    d = sg.probe(a, b, c, dt)
    want = sg.model(a, b, c, dt)
    exact = float(np.mean(d.view(np.uint32) == want.view(np.uint32)))
    if OUT.is_dir():
        (OUT / f"mfma_step_{dt}_{kind}.json").write_text(json.dumps({"dtype": dt, "kind": kind, "exact": exact}))
    assert_bits_equal(d, want, f"{dt} {kind}")


def test_committed_step_fixture_reproduces_on_this_gpu():
    """The single-step vectors in tests/golden/mfma_step_gfx950.npz come back
    bit for bit from this GPU (the CPU suite checks the oracle against the
    same file)."""
    fx = np.load(sg.FIXTURE)
    for dt in sg.DTYPES:
        for kind in sg.KINDS:
            a, b, c = sg.step_operands(dt, kind, sg.FIXTURE_SEED)
            assert_bits_equal(sg.probe(a, b, c, dt), fx[f"{dt}_{kind}"], f"{dt} {kind}")
