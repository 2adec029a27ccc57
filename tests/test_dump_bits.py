"""Bit-hash dump / compare tool (mlx_batch_invariant_amd.dump_bits): the
compare report on hand-made dumps (CPU), and a real dump on the GPU, which
must reproduce itself within one process and cover every op, dtype and mode."""

import io
import json

import pytest

from mlx_batch_invariant_amd import dump_bits as db


def _d(ops, model=None, **meta):
    return {"torch": "t", "hip": "h", "device": "d", "arch": "gfx950", "library": "x", **meta,
            "ops": ops, "model": model or {}}


def test_compare_counts_and_exit_code():
    a = _d({"matmul/bf16/inv": "1", "matmul/bf16/stock": "2", "rms_norm/fp32/inv": "3"})
    b = _d({"matmul/bf16/inv": "1", "matmul/bf16/stock": "9", "rms_norm/fp32/inv": "3"})
    buf = io.StringIO()
    assert db.compare(a, b, file=buf) == 0        # only a stock hash differs
    text = buf.getvalue()
    assert "[ops] inv: 2 of 2 hashes agree" in text and "[ops] stock: 0 of 1 hashes agree" in text
    assert "differ: matmul/bf16/stock" in text and "invariant hashes agree" in text
    buf = io.StringIO()
    assert db.compare(a, _d({"matmul/bf16/inv": "1", "extra/f16/inv": "4"}), file=buf) == 0
    assert "in one dump only: extra/f16/inv, matmul/bf16/stock, rms_norm/fp32/inv" in buf.getvalue()
    c = _d({"matmul/bf16/inv": "7", "matmul/bf16/stock": "2", "rms_norm/fp32/inv": "3"})
    assert db.compare(a, c, file=io.StringIO()) == 1   # an invariant hash differs


def test_compare_cli(tmp_path):
    a, b = tmp_path / "a.json", tmp_path / "b.json"
    a.write_text(json.dumps(_d({"matmul/bf16/inv": "1"}, {"llama2-bf16/decode/inv": "5"})))
    b.write_text(json.dumps(_d({"matmul/bf16/inv": "1"}, {"llama2-bf16/decode/inv": "6"})))
    assert db.main(["--compare", str(a), str(b)]) == 1
    with pytest.raises(SystemExit):
        db.main([])


@pytest.mark.gpu
def test_dump_reproduces_itself(tmp_path):
    out = tmp_path / "bits.json"
    assert db.main(["--out", str(out), "--model", "llama:1"]) == 0
    d1 = json.loads(out.read_text())
    d2 = db.dump("llama:1")
    names = {"matmul", "addmm", "qmatmul_4b", "qmatmul_8b", "rms_norm", "sdpa_decode", "sdpa_prefill"}
    assert {k.split("/")[0] for k in d1["ops"]} == names
    assert len(d1["ops"]) == len(names) * 3 * 2 and len(d1["model"]) == 2 * 2 * 2
    assert d1["ops"] == d2["ops"] and d1["model"] == d2["model"]
    assert db.compare(d1, d2, file=io.StringIO()) == 0


@pytest.mark.gpu
def test_dump_invariant_hashes_equal_the_oracles_bits():
    """Every invariant-mode op hash of a dump equals the hash of the oracle's
    output on the same probe inputs (the dump's own CPU draws): matmul, addmm
    (matmul rounded, then + bias rounded), 4-bit and 8-bit quantized matmul
    (the blocked k-slot map), RMSNorm, and decode / causal prefill attention
    (the matrix-core emulation with the hardware exp2), in fp16, bf16, fp32."""
    import numpy as np
    import torch

    from helpers import gpu_exp2
    from oracle import bi_oracle as ora
    d = db.dump()
    names = {torch.float16: ("fp16", "f16"), torch.bfloat16: ("bf16", "bf16"), torch.float32: ("fp32", "f32")}
    f = lambda t: t.float().numpy()
    for dt, (tag, o) in names.items():
        p = db.probe_inputs(dt)
        x, W = f(p["x"]), f(p["W"])
        mm = ora.matmul(x, W, o)
        want = {"matmul": mm, "addmm": ora.round_to((mm + f(p["lin_b"])).astype(np.float32), o)}
        for name, bits_, gs in db.QUANT:
            wq, s, b = p[name]
            Wd = ora.dequantize(wq.numpy().view(np.uint32), f(s), f(b), gs, bits_, o)
            want[name] = ora.matmul(x, Wd, o, kmap="blocked")
        want["rms_norm"] = ora.rms_norm(f(p["x_n"]), f(p["w_n"]), 1e-5, o)
        want["sdpa_decode"] = ora.attention_mfma(f(p["q"]), f(p["k"]), f(p["v"]), db.DH ** -0.5, False, o,
                                                 exp2=gpu_exp2)
        want["sdpa_prefill"] = ora.attention_mfma(f(p["qp"]), f(p["kp"]), f(p["vp"]), db.DH ** -0.5, True, o,
                                                  exp2=gpu_exp2)
        for name, arr in want.items():
            h = db.hash_array(torch.from_numpy(np.ascontiguousarray(arr, np.float32)).to(dt))
            assert d["ops"][f"{name}/{tag}/inv"] == h, f"{name}/{tag}"
