"""Batch-sweep conformance report: stock torch against the batch-invariant mode.

    python -m mlx_batch_invariant_amd.conformance [--ops ...] [--dtypes ...]
        [--batch-sizes ...] [--strict] [--json out.json]

Counterpart of mlx-batch-invariant's harness/sweep.py (:224-289, report
format of harness/last_sweep.txt). For each (op, dtype) a fixed probe row is
embedded at the first and the last position of batches of increasing size and
compared bit for bit with its batch-1 result, once with the stock torch ops
(hipBLASLt / rocBLAS matmul, F.rms_norm, F.scaled_dot_product_attention,
dequantize + matmul for the affine quantized format) and once inside
``set_batch_invariant_mode``. "FAIL @B=n" names the smallest batch whose probe
row differs; max|diff| is over the whole sweep. Then the attention structure
checks: chunked prefill == one-shot prefill and decode(last) == prefill(last).

Ops and shapes are the reference harness's (harness/sweep.py:65-179):
matmul / addmm x[B, 4096] @ W[4096, 4096]^T (addmm with a bias), 4-bit g64 and
8-bit g32 quantized matmul of the same W, RMSNorm over 4096 (eps 1e-5),
decode attention 8 / 2 heads of 128 over 1000 keys, causal prefill of 48
tokens against 300 keys. Probe rows and weights come from a fixed CPU
generator; filler rows from a device generator seeded per (batch, position).
"""

from __future__ import annotations

import argparse
import json
import sys
from dataclasses import asdict, dataclass, field

import torch

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
DEFAULT_BATCHES = [1, 2, 3, 4, 8, 16, 32, 64, 128, 256]


def _bits(t) -> bytes:
    if isinstance(t, tuple):
        return b"".join(_bits(x) for x in t)
    return t.detach().contiguous().view(torch.uint8).cpu().numpy().tobytes()


def _maxdiff(a, b) -> float:
    return float((a.float() - b.float()).abs().max())


class _Op:
    """A probe row (or tuple of rows) and a run(batch) -> output, axis 0 = batch."""
    name = ""

    def __init__(self, dt, seed: int):
        self.dt = dt
        self.g = torch.Generator().manual_seed(seed)
        self.setup()

    def rn(self, *shape):
        return torch.randn(shape, generator=self.g).to(self.dt).cuda()

    def setup(self):
        raise NotImplementedError

    def filler(self, n: int, gd: torch.Generator):
        """n rows of the probe's shape, drawn on the device."""
        if isinstance(self.probe, tuple):
            return tuple(torch.randn((n, *p.shape[1:]), generator=gd, device="cuda").to(self.dt) for p in self.probe)
        return torch.randn((n, *self.probe.shape[1:]), generator=gd, device="cuda").to(self.dt)

    def run(self, batch):
        raise NotImplementedError


class Matmul(_Op):
    name = "matmul"
    K = N = 4096

    def setup(self):
        self.W = self.rn(self.N, self.K)              # nn.Linear layout
        self.probe = self.rn(1, self.K)

    def run(self, x):
        return torch.matmul(x, self.W.t())


class Addmm(Matmul):
    name = "addmm"

    def setup(self):
        super().setup()
        self.b = self.rn(self.N)

    def run(self, x):
        return torch.nn.functional.linear(x, self.W, self.b)


class QuantizedMatmul(Matmul):
    name = "qmatmul_4b"
    bits, gs = 4, 64

    def setup(self):
        from .kernels.quantized import quantize
        super().setup()
        wq, s, b = quantize(self.W.float().cpu(), group_size=self.gs, bits=self.bits, dtype=self.dt)
        self.wq, self.s, self.b = wq.view(torch.int32).cuda(), s.cuda(), b.cuda()

    def run(self, x):
        from . import nn as bnn
        return bnn.quantized_matmul(x, self.wq, self.s, self.b, transpose=True, group_size=self.gs, bits=self.bits)


class QuantizedMatmul8(QuantizedMatmul):
    name = "qmatmul_8b"
    bits, gs = 8, 32


class RMSNorm(_Op):
    name = "rms_norm"
    D = 4096

    def setup(self):
        self.w = self.rn(self.D)
        self.probe = self.rn(1, self.D)

    def run(self, x):
        return torch.nn.functional.rms_norm(x, (self.D,), self.w, 1e-5)


class SDPADecode(_Op):
    name = "sdpa_decode"
    Hq, Hkv, L, D = 8, 2, 1000, 128

    def setup(self):
        self.probe = (self.rn(1, self.Hq, 1, self.D), self.rn(1, self.Hkv, self.L, self.D),
                      self.rn(1, self.Hkv, self.L, self.D))

    def run(self, b):
        q, k, v = b
        return torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=self.D ** -0.5, enable_gqa=True)


class SDPAPrefill(_Op):
    name = "sdpa_prefill"
    Hq, Hkv, Tq, L, D = 8, 2, 48, 300, 128           # L > Tq: causal against a cache

    def setup(self):
        self.probe = (self.rn(1, self.Hq, self.Tq, self.D), self.rn(1, self.Hkv, self.L, self.D),
                      self.rn(1, self.Hkv, self.L, self.D))

    def run(self, b):
        from torch.nn.attention.bias import causal_lower_right
        q, k, v = b
        return torch.nn.functional.scaled_dot_product_attention(
            q, k, v, attn_mask=causal_lower_right(self.Tq, self.L), scale=self.D ** -0.5, enable_gqa=True)


OPS = {c.name: c for c in (Matmul, Addmm, QuantizedMatmul, QuantizedMatmul8, RMSNorm, SDPADecode, SDPAPrefill)}


@dataclass
class Result:
    op: str
    dtype: str
    mode: str
    passed: bool = True
    first_fail: int | None = None
    max_diff: float = 0.0
    fallbacks: dict = field(default_factory=dict)


def _embed(op: _Op, B: int, pos: int, seed: int):
    gd = torch.Generator(device="cuda").manual_seed(seed + 7 * B + pos)
    parts = []
    if pos > 0:
        parts.append(op.filler(pos, gd))
    parts.append(op.probe)
    if B - 1 - pos > 0:
        parts.append(op.filler(B - 1 - pos, gd))
    if isinstance(op.probe, tuple):
        return tuple(torch.cat([p[i] for p in parts], 0) for i in range(len(op.probe)))
    return torch.cat(parts, 0)


def sweep_one(op: _Op, batches, invariant: bool, seed: int = 0) -> Result:
    import mlx_batch_invariant_amd as bi
    res = Result(op.name, next(k for k, v in DTYPES.items() if v == op.dt), "INVARIANT" if invariant else "STOCK")
    bi.reset_stats()
    with bi.set_batch_invariant_mode(enabled=invariant):
        ref = op.run(op.probe)[0:1]
        ref_bits = _bits(ref)
        for B in batches:
            for pos in sorted({0, B - 1}):
                out = op.run(_embed(op, B, pos, seed))[pos:pos + 1]
                if _bits(out) != ref_bits:
                    res.passed = False
                    res.first_fail = res.first_fail or B
                    res.max_diff = max(res.max_diff, _maxdiff(out, ref))
    res.fallbacks = {k: v for k, v in bi.stats()["fallbacks"].items() if v}
    return res


def structure_checks(dt, invariant: bool, seed: int = 0) -> dict:
    """Chunked == one-shot prefill and decode(last) == prefill(last), 8 / 2
    heads of 128, T = 600, first chunk 257 tokens (not a multiple of the
    256-key split)."""
    import mlx_batch_invariant_amd as bi
    from torch.nn.attention.bias import causal_lower_right
    Hq, Hkv, D, T, T1 = 8, 2, 128, 600, 257
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(s, generator=g).to(dt).cuda()
    q, k, v = r(2, Hq, T, D), r(2, Hkv, T, D), r(2, Hkv, T, D)
    F = torch.nn.functional
    sd = lambda q_, k_, v_, **kw: F.scaled_dot_product_attention(q_, k_, v_, scale=D ** -0.5, enable_gqa=True, **kw)
    with bi.set_batch_invariant_mode(enabled=invariant):
        full = sd(q, k, v, is_causal=True)
        p1 = sd(q[:, :, :T1], k[:, :, :T1], v[:, :, :T1], is_causal=True)
        p2 = sd(q[:, :, T1:], k, v, attn_mask=causal_lower_right(T - T1, T))
        dec = sd(q[:, :, T - 1:T], k, v)
    return {"chunked_prefill == full_prefill": _bits(torch.cat([p1, p2], 2)) == _bits(full),
            "decode(last) == prefill(last)": _bits(dec) == _bits(full[:, :, T - 1:T])}


def fmt(r: Result) -> str:
    status = "pass" if r.passed else f"FAIL @B={r.first_fail} max|diff|={r.max_diff:.3g}"
    fb = f"  fallbacks={r.fallbacks}" if r.fallbacks else ""
    return f"{r.op:<12} {r.dtype:<9} {r.mode:<10} {status}{fb}"


def run(ops=None, dtypes=None, batches=None, seed: int = 0, file=sys.stdout) -> dict:
    """Print the report; return it as a dict (rows, structure checks, verdict)."""
    ops = ops or list(OPS)
    dtypes = dtypes or list(DTYPES)
    batches = batches or DEFAULT_BATCHES
    props = torch.cuda.get_device_properties(0)
    print(f"torch {torch.__version__} (HIP {getattr(torch.version, 'hip', None)}) on {props.name} "
          f"({getattr(props, 'gcnArchName', '?')})", file=file)
    print(f"batch sizes: {batches}\n", file=file)
    print(f"{'op':<12} {'dtype':<9} {'mode':<10} result", file=file)
    print("-" * 64, file=file)
    rows, inv_fail = [], False
    for op_name in ops:
        for dt_name in dtypes:
            op = OPS[op_name](DTYPES[dt_name], seed)
            for invariant in (False, True):
                r = sweep_one(op, batches, invariant, seed)
                rows.append(asdict(r))
                print(fmt(r), file=file, flush=True)
                inv_fail |= invariant and not r.passed
            del op
    print("\nattention structure checks (chunked prefill, decode vs prefill):", file=file)
    checks = []
    for dt_name in dtypes:
        for invariant in (False, True):
            mode = "INVARIANT" if invariant else "STOCK"
            for name, ok in structure_checks(DTYPES[dt_name], invariant, seed).items():
                checks.append({"dtype": dt_name, "mode": mode, "check": name, "passed": ok})
                print(f"{'sdpa':<12} {dt_name:<9} {mode:<10} {name}: {'pass' if ok else 'FAIL'}", file=file)
                inv_fail |= invariant and not ok
    print("", file=file)
    print("INVARIANT mode FAILED somewhere above." if inv_fail else
          "INVARIANT mode: all probe rows bitwise identical across the sweep.", file=file)
    return {"batches": batches, "rows": rows, "structure": checks, "invariant_all_pass": not inv_fail}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--ops", nargs="+", default=list(OPS), choices=list(OPS))
    p.add_argument("--dtypes", nargs="+", default=list(DTYPES), choices=list(DTYPES))
    p.add_argument("--batch-sizes", nargs="+", type=int, default=DEFAULT_BATCHES)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--strict", action="store_true", help="exit 1 if the invariant mode fails anywhere")
    p.add_argument("--json", default=None, help="also write the report as JSON to this path")
    a = p.parse_args(argv)
    rep = run(a.ops, a.dtypes, a.batch_sizes, a.seed)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rep, f, indent=1)
    return 1 if (a.strict and not rep["invariant_all_pass"]) else 0


if __name__ == "__main__":
    sys.exit(main())
