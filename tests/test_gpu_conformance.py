"""The conformance sweep report (mlx_batch_invariant_amd.conformance, the
reference's harness/sweep.py) on the GPU: the invariant mode passes every op x
dtype over batches 1-256 and both structure checks; the stock rows are
recorded, not asserted (they are the evidence that stock torch diverges)."""

import io
import json
import os
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu


def test_conformance_sweep_invariant_mode_passes_everywhere():
    from mlx_batch_invariant_amd import conformance
    buf = io.StringIO()
    rep = conformance.run(file=buf)
    text = buf.getvalue()
    out = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"
    if out.is_dir():
        (out / "conformance_sweep.txt").write_text(text)
        (out / "conformance_sweep.json").write_text(json.dumps(rep, indent=1))
    inv = [r for r in rep["rows"] if r["mode"] == "INVARIANT"]
    assert len(inv) == len(conformance.OPS) * len(conformance.DTYPES)
    bad = [r for r in inv if not r["passed"] or r["fallbacks"]]
    assert not bad, bad
    assert all(c["passed"] for c in rep["structure"] if c["mode"] == "INVARIANT"), rep["structure"]
    assert rep["invariant_all_pass"]
    assert "INVARIANT mode: all probe rows bitwise identical across the sweep." in text
