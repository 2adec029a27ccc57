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

from helpers import bits, gpu_exp2

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


def _np_forward(model, tokens):
    """A numpy forward of one sequence's prefill built from the oracle
    (rms_norm, dequantize, matmul with the quantized k-slot map, the per-key
    attention) and torch's bf16 elementwise rounding (each elementwise op is
    computed in fp32 and rounded once to bf16). Returns (row-0 hidden after the
    first norm, its Q projection, the last token's logits)."""
    import numpy as np
    from oracle import bi_oracle as ora
    cfg = model.cfg
    rb = lambda a: ora.round_to(np.asarray(a, np.float32), "bf16")
    f = lambda t: t.detach().float().cpu().numpy()

    def lin(layer, x):
        if cfg.bits is None:
            return ora.matmul(x, f(layer.weight), "bf16")
        W = ora.dequantize(layer.weight.cpu().numpy().view(np.uint32), f(layer.scales), f(layer.biases),
                           layer.group_size, layer.bits, "bf16")
        return ora.matmul(x, W, "bf16", kmap="blocked")

    T = tokens.shape[0]
    x = f(model.embed)[tokens]
    cos, sin = (f(t) for t in model._rope_tables(0, T))

    def rope(h):                                                  # h [H, T, D]
        d2 = h.shape[-1] // 2
        x1, x2 = h[..., :d2], h[..., d2:]
        return np.concatenate([rb(rb(x1 * cos) - rb(x2 * sin)), rb(rb(x2 * cos) + rb(x1 * sin))], -1)

    first = None
    for blk in model.blocks:
        hn = ora.rms_norm(x, f(blk.attn_norm.weight), cfg.eps, "bf16")
        q = lin(blk.q, hn)
        if first is None:
            first = (hn, q)
        q = rope(q.reshape(T, cfg.heads, cfg.head_dim).transpose(1, 0, 2))
        k = rope(lin(blk.k, hn).reshape(T, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2))
        v = lin(blk.v, hn).reshape(T, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
        a = ora.attention_mfma(q[None], k[None], v[None], cfg.head_dim ** -0.5, True, "bf16", exp2=gpu_exp2)[0]
        x = rb(x + lin(blk.o, a.transpose(1, 0, 2).reshape(T, -1)))
        hn = ora.rms_norm(x, f(blk.mlp_norm.weight), cfg.eps, "bf16")
        g = lin(blk.gate, hn)
        silu = rb(g / (np.float32(1) + np.exp(-g)))
        x = rb(x + lin(blk.down, rb(silu * lin(blk.up, hn))))
    hl = ora.rms_norm(x[-1:], f(model.norm.weight), cfg.eps, "bf16")
    return first, lin(model.head, hl)[0]


@pytest.mark.parametrize("bits_", [4, None], ids=["q4g64", "bf16"])
def test_forward_matches_numpy_oracle_forward(bits_):
    """Oracle anchor of the model path: a 1-layer Llama-shaped decoder with
    reduced widths (hidden 512, MLP 1536, 4 / 2 heads of 128, vocab 1000),
    prefill of 24 tokens under the mode, against a numpy forward built from
    the oracle's functions (attention: the emulation of the matrix-core order
    with the hardware exp2; RoPE, residual adds and SiLU as torch rounds them
    in bf16). The first norm and Q projection and the logits are bit-exact."""
    import numpy as np
    import mlx_batch_invariant_amd as bi
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    cfg = LlamaConfig(layers=1, hidden=512, ffn=1536, heads=4, kv_heads=2, head_dim=128, vocab=1000, bits=bits_)
    model = LlamaShaped(cfg, device="cuda", dtype=torch.bfloat16, seed=5)
    toks = torch.randint(0, cfg.vocab, (1, 24), generator=torch.Generator().manual_seed(9)).cuda()
    with bi.set_batch_invariant_mode(strict=True):
        logits = model(toks, model.new_cache(1, 24), 0)
        blk = model.blocks[0]
        hn = blk.attn_norm(model.embed[toks[0]])
        q = blk.q(hn)
    (hn_np, q_np), want = _np_forward(model, toks[0].cpu().numpy())
    f = lambda t: t.detach().float().cpu().numpy()
    assert np.array_equal(f(hn), hn_np)
    assert np.array_equal(f(q), q_np)
    got = f(logits)[0]
    rel = float(np.abs(got - want).max() / np.abs(want).max())
    exact = float(np.mean(got == want))
    if OUT.is_dir():
        (OUT / f"llama_oracle_anchor_{bits_ or 'bf16'}.json").write_text(json.dumps({"max_rel": rel, "exact": exact}))
    assert exact == 1.0, (rel, exact)
