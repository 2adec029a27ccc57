"""BASELINE config 5 at its configured size: the 32-layer Llama-3-8B-shape
decoder (hidden 4096, MLP 14336, 32 query / 8 KV heads of 128, vocab 128256,
RoPE theta 5e5), 4-bit affine g64 linears and bf16 linears, a 512-token
random prompt then 128 greedy decode steps at batch 1, 4, 16 and 64, in
strict invariant mode (no fallback).

Row 0 holds the same prompt at every batch size: its logits at all 129 steps
(the prefill's last token and every decode step) must be bitwise identical
across batch sizes, and so must the greedy tokens. One-shot prefill must equal
chunked prefill (chunks of 128 over a 512-token prompt; chunks of 512 over a
1024-token prompt), bit for bit, in the logits and in every KV cache.
Reference protocol: harness/model_sweep.py:62-108 (row-0 recorder),
harness/generate_bench.py:24-71 (prefill + greedy steps).
"""

import json
import os
import time
from pathlib import Path

import pytest
import torch

from helpers import bits

pytestmark = pytest.mark.gpu

OUT = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"
BATCHES = (1, 4, 16, 64)
T_PROMPT, STEPS = 512, 128


@pytest.fixture(scope="module", params=[4, None], ids=["q4g64", "bf16"])
def full_model(request):
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    t0 = time.perf_counter()
    m = LlamaShaped(LlamaConfig(layers=32, bits=request.param), device="cuda", dtype=torch.bfloat16, seed=0)
    torch.cuda.synchronize()
    print(f"built {request.param or 'bf16'} model in {time.perf_counter() - t0:.1f} s", flush=True)
    yield m
    del m
    torch.cuda.empty_cache()


def _prompt(B, vocab, T=T_PROMPT):
    row0 = torch.randint(0, vocab, (1, T), generator=torch.Generator().manual_seed(0))
    fill = torch.randint(0, vocab, (B - 1, T), generator=torch.Generator().manual_seed(B))
    return torch.cat([row0, fill], 0).cuda()


def test_config5_row0_logits_bitwise_across_batch_sizes(full_model):
    import mlx_batch_invariant_amd as bi
    bi.reset_stats()
    ref = None
    timing = {}
    with bi.set_batch_invariant_mode(strict=True):
        for B in BATCHES:
            t0 = time.perf_counter()
            logits, toks = full_model.generate(_prompt(B, full_model.cfg.vocab), STEPS)
            torch.cuda.synchronize()
            timing[B] = round(time.perf_counter() - t0, 2)
            got = (bits(logits), toks[0].cpu())
            assert logits.shape == (STEPS + 1, full_model.cfg.vocab)
            if ref is None:
                ref = got
            else:
                assert got[0] == ref[0], f"B={B}: row-0 logits differ from B=1"
                assert torch.equal(got[1], ref[1]), f"B={B}: row-0 greedy tokens differ from B=1"
            print(f"B={B}: prefill {T_PROMPT} + {STEPS} steps in {timing[B]} s", flush=True)
    st = bi.stats()
    assert not st["fallbacks"], st
    tag = f"q{full_model.cfg.bits}" if full_model.cfg.bits else "bf16"
    if OUT.is_dir():
        (OUT / f"llama_full_{tag}.json").write_text(json.dumps({"seconds_by_batch": timing, "handled": st["handled"]}))


def test_config5_chunked_prefill_equals_one_shot(full_model):
    import mlx_batch_invariant_amd as bi
    B = 2
    with bi.set_batch_invariant_mode(strict=True):
        for T, C in ((T_PROMPT, 128), (2 * T_PROMPT, 512)):
            toks = _prompt(B, full_model.cfg.vocab, T)
            c1 = full_model.new_cache(B, T)
            one = full_model(toks, c1, 0)
            c2 = full_model.new_cache(B, T)
            for s in range(0, T, C):
                chunked = full_model(toks[:, s:s + C], c2, s)
            torch.cuda.synchronize()
            assert bits(one) == bits(chunked), (T, C)
            for li, ((k1, v1), (k2, v2)) in enumerate(zip(c1, c2)):
                assert bits(k1) == bits(k2) and bits(v1) == bits(v2), (T, C, li)
            del c1, c2
