"""A random-initialised Llama-3-8B-shaped decoder built from stock torch
modules, used to check that the four batch-invariant ops compose.

Every matmul goes through ``nn.Linear`` / ``F.linear`` (or this package's
``QuantizedLinear`` for MLX-affine weights), every norm through ``nn.RMSNorm``
and attention through ``F.scaled_dot_product_attention``, so the model is the
stock path outside ``set_batch_invariant_mode`` and the batch-invariant kernels
inside it, with no code change: the drop-in property the reference checks
end to end with ``harness/model_sweep.py`` (row-0 logits / per-block hashes at
batch 1, 4, 16, 64, prefill and cached decode; :62-108).

Prefill is causal over the prompt (``is_causal``; a later chunk of a chunked
prefill uses ``causal_lower_right``); decode steps attend to a preallocated KV
cache through a view (no copy), one token per sequence. RoPE (theta 5e5),
SiLU-gated MLP and residual adds are elementwise torch ops, which compute each
element from its own inputs only.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

from .nn import QuantizedLinear


@dataclass
class LlamaConfig:
    vocab: int = 128256
    hidden: int = 4096
    ffn: int = 14336
    layers: int = 32
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    rope_theta: float = 5e5
    eps: float = 1e-5
    bits: int | None = 4          # None: bf16 linears
    group_size: int = 64


def _linear(cfg: LlamaConfig, fin: int, fout: int, gen: torch.Generator, device, dtype):
    """``nn.Linear`` (bf16 run) or ``QuantizedLinear`` quantized from it, with
    N(0, 0.02^2) weights drawn on ``device``."""
    lin = torch.nn.Linear(fin, fout, bias=False, device="meta", dtype=dtype)
    w = (torch.randn((fout, fin), generator=gen, device=device) * 0.02).to(dtype)
    lin.weight = torch.nn.Parameter(w, requires_grad=False)
    if cfg.bits is None:
        return lin
    q = QuantizedLinear.from_linear(lin, group_size=cfg.group_size, bits=cfg.bits)
    del lin, w
    return q


class Block(torch.nn.Module):
    def __init__(self, cfg: LlamaConfig, gen, device, dtype):
        super().__init__()
        h, kvd = cfg.hidden, cfg.kv_heads * cfg.head_dim
        self.cfg = cfg
        self.attn_norm = torch.nn.RMSNorm(h, eps=cfg.eps, device=device, dtype=dtype)
        self.mlp_norm = torch.nn.RMSNorm(h, eps=cfg.eps, device=device, dtype=dtype)
        self.q = _linear(cfg, h, cfg.heads * cfg.head_dim, gen, device, dtype)
        self.k = _linear(cfg, h, kvd, gen, device, dtype)
        self.v = _linear(cfg, h, kvd, gen, device, dtype)
        self.o = _linear(cfg, cfg.heads * cfg.head_dim, h, gen, device, dtype)
        self.gate = _linear(cfg, h, cfg.ffn, gen, device, dtype)
        self.up = _linear(cfg, h, cfg.ffn, gen, device, dtype)
        self.down = _linear(cfg, cfg.ffn, h, gen, device, dtype)

    def forward(self, x, cos, sin, cache, pos):
        cfg = self.cfg
        B, T, _ = x.shape
        hn = self.attn_norm(x)
        q = self.q(hn).view(B, T, cfg.heads, cfg.head_dim).transpose(1, 2)
        k = self.k(hn).view(B, T, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        v = self.v(hn).view(B, T, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        q = _rope(q, cos, sin)
        k = _rope(k, cos, sin)
        kc, vc = cache
        kc[:, :, pos:pos + T] = k
        vc[:, :, pos:pos + T] = v
        L = pos + T
        if T == 1:
            mask = {}
        elif pos == 0:
            mask = {"is_causal": True}
        else:                                   # chunked prefill: chunk t sees keys <= pos + t
            mask = {"attn_mask": causal_lower_right(T, L)}
        a = F.scaled_dot_product_attention(q, kc[:, :, :L], vc[:, :, :L], enable_gqa=True, **mask)
        x = x + self.o(a.transpose(1, 2).reshape(B, T, cfg.heads * cfg.head_dim))
        hn = self.mlp_norm(x)
        x = x + self.down(F.silu(self.gate(hn)) * self.up(hn))
        return x


def _rope(x, cos, sin):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


class LlamaShaped(torch.nn.Module):
    """Decoder with Llama-3-8B shapes (or fewer layers for tests)."""

    def __init__(self, cfg: LlamaConfig, device="cuda", dtype=torch.bfloat16, seed: int = 0):
        super().__init__()
        gen = torch.Generator(device=device).manual_seed(seed)
        self.cfg = cfg
        self.dtype = dtype
        self.embed = (torch.randn((cfg.vocab, cfg.hidden), generator=gen, device=device) * 0.02).to(dtype)
        self.blocks = torch.nn.ModuleList([Block(cfg, gen, device, dtype) for _ in range(cfg.layers)])
        self.norm = torch.nn.RMSNorm(cfg.hidden, eps=cfg.eps, device=device, dtype=dtype)
        self.head = _linear(cfg, cfg.hidden, cfg.vocab, gen, device, dtype)
        self.device = torch.device(device)

    def _ensure_rope(self, n: int):
        """cos / sin tables of positions [0, n) on the device (built once, grown
        on demand outside any graph capture; every position's entries are
        computed from that position alone, so a slice equals a fresh table)."""
        have = getattr(self, "_rope_cos", None)
        if have is not None and have.shape[0] >= n:
            return
        cfg = self.cfg
        n = max(n, 2 * (have.shape[0] if have is not None else 0))
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float64) / cfg.head_dim))
        ang = torch.outer(torch.arange(0, n, dtype=torch.float64), inv)
        self._rope_cos = ang.cos().to(self.dtype).to(self.device)
        self._rope_sin = ang.sin().to(self.dtype).to(self.device)

    def _rope_tables(self, pos, T):
        self._ensure_rope(pos + T)
        return self._rope_cos[pos:pos + T], self._rope_sin[pos:pos + T]

    def new_cache(self, B: int, max_len: int):
        cfg = self.cfg
        self._ensure_rope(max_len)
        shape = (B, cfg.kv_heads, max_len, cfg.head_dim)
        return [(torch.zeros(shape, dtype=self.dtype, device=self.device),
                 torch.zeros(shape, dtype=self.dtype, device=self.device)) for _ in range(cfg.layers)]

    @torch.no_grad()
    def forward(self, tokens, cache, pos: int, record=None):
        x = self.embed[tokens]
        cos, sin = self._rope_tables(pos, tokens.shape[1])
        for i, blk in enumerate(self.blocks):
            x = blk(x, cos, sin, cache[i], pos)
            if record is not None:
                record.append(x[0:1, -1:].clone())
        return self.head(self.norm(x[:, -1:]))[:, 0]

    @torch.no_grad()
    def generate(self, prompt, steps: int, record=None):
        """Greedy: prefill the prompt, then `steps` cached decode steps.
        Returns (logits of every step [steps+1, B, vocab] for row 0 only, tokens)."""
        B, T = prompt.shape
        cache = self.new_cache(B, T + steps)
        logits = self.forward(prompt, cache, 0, record)
        rows0 = [logits[0:1].clone()]
        tok = logits.argmax(-1, keepdim=True)
        out = [tok]
        for s in range(steps):
            logits = self.forward(tok, cache, T + s, record)
            rows0.append(logits[0:1].clone())
            tok = logits.argmax(-1, keepdim=True)
            out.append(tok)
        return torch.cat(rows0, 0), torch.cat(out, 1)


def param_bytes(model: LlamaShaped) -> int:
    n = 0
    for t in list(model.parameters()) + list(model.buffers()):
        n += t.numel() * t.element_size()
    return n + model.embed.numel() * model.embed.element_size()
