"""End-to-end invariance of a Llama-3-8B-shaped decoder under the mode
(reference protocol: harness/model_sweep.py:62-108 and the decode variant
:88-96; the reference runs it on a downloaded bf16 checkpoint, here the
weights are random and the widths are Llama-3-8B's: hidden 4096, 32 query /
8 KV heads of 128, MLP 14336, vocab 128256, with 2 of the 32 blocks).

Row 0 holds a fixed prompt, the other rows random tokens. Every block's row-0
output and the row-0 logits of the prefill and of each greedy decode step must
be bitwise identical at batch 1, 4, 16 and 64, with no fallback (strict mode).
Chunked prefill must equal one-shot prefill, and the decode step for position
t must equal the prefill's output at t.
"""

import json
import os
from pathlib import Path

import pytest
import torch

from helpers import bits

pytestmark = pytest.mark.gpu

OUT = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"
BATCHES = (1, 4, 16, 64)
T_PROMPT = 20
STEPS = 3


def _model(bits_):
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    cfg = LlamaConfig(layers=2, bits=bits_)
    return LlamaShaped(cfg, device="cuda", dtype=torch.bfloat16, seed=3)


@pytest.fixture(scope="module", params=[4, None], ids=["q4g64", "bf16"])
def model(request):
    m = _model(request.param)
    yield m
    del m
    torch.cuda.empty_cache()


def _tokens(B, vocab, seed=0):
    g = torch.Generator().manual_seed(1234)
    row0 = torch.randint(0, vocab, (1, T_PROMPT), generator=g)
    g2 = torch.Generator().manual_seed(seed + B)
    fill = torch.randint(0, vocab, (B - 1, T_PROMPT), generator=g2)
    return torch.cat([row0, fill], 0).cuda()


def _run(model, B):
    rec = []
    logits, toks = model.generate(_tokens(B, model.cfg.vocab), STEPS, record=rec)
    torch.cuda.synchronize()
    return [bits(r) for r in rec], bits(logits), toks[0].cpu()


def test_row0_bitwise_across_batch_sizes(model):
    import mlx_batch_invariant_amd as bi
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        ref_blocks, ref_logits, ref_toks = _run(model, 1)
        for B in BATCHES[1:]:
            blocks, logits, toks = _run(model, B)
            first_bad = next((i for i, (a, b) in enumerate(zip(ref_blocks, blocks)) if a != b), None)
            assert first_bad is None, f"B={B}: row-0 output of forward/block {first_bad} differs from B=1"
            assert ref_logits == logits, f"B={B}: row-0 logits differ"
            assert torch.equal(ref_toks, toks)
    st = bi.stats()
    assert not st["fallbacks"], st
    h = st["handled"]
    assert h.get("rms_norm", 0) > 0 and h.get("sdpa_prefill", 0) > 0 and h.get("sdpa_decode", 0) > 0
    assert h.get("quantized_matmul" if model.cfg.bits else "matmul", 0) > 0


def test_stock_path_report(model):
    """Records whether the stock ROCm path is batch-variant on this model
    (informational, as the reference's sweep prints STOCK diverging)."""
    ref_blocks, ref_logits, _ = _run(model, 1)
    report = {}
    for B in BATCHES[1:]:
        blocks, logits, _ = _run(model, B)
        bad = [i for i, (a, b) in enumerate(zip(ref_blocks, blocks)) if a != b]
        report[B] = {"first_divergent_forward_block": bad[0] if bad else None,
                     "logits_equal": ref_logits == logits}
    tag = f"q{model.cfg.bits}" if model.cfg.bits else "bf16"
    if OUT.is_dir():
        (OUT / f"llama_stock_divergence_{tag}.json").write_text(json.dumps(report, indent=1))
    print(tag, report)


def test_chunked_prefill_and_decode_match_one_shot(model):
    import mlx_batch_invariant_amd as bi
    B = 4
    toks = _tokens(B, model.cfg.vocab)
    with bi.set_batch_invariant_mode(strict=True):
        c1 = model.new_cache(B, T_PROMPT)
        one = model(toks, c1, 0)                                  # prefill of all T tokens
        c2 = model.new_cache(B, T_PROMPT)
        model(toks[:, :13], c2, 0)
        chunked = model(toks[:, 13:], c2, 13)                     # second chunk over the cache
        c3 = model.new_cache(B, T_PROMPT)
        model(toks[:, :-1], c3, 0)
        decoded = model(toks[:, -1:], c3, T_PROMPT - 1)           # last token as a decode step
        torch.cuda.synchronize()
    assert bits(one) == bits(chunked)
    assert bits(one) == bits(decoded)
    for (k1, v1), (k2, v2), (k3, v3) in zip(c1, c2, c3):
        assert bits(k1) == bits(k2) and bits(v1) == bits(v2)
        assert bits(k1) == bits(k3) and bits(v1) == bits(v3)
