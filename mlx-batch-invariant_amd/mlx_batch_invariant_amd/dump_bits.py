"""Bit hashes of the invariant kernels' outputs (and a model's logits), so two
software stacks or two machines can be compared.

    python -m mlx_batch_invariant_amd.dump_bits --out bits_<tag>.json [--model llama[:LAYERS]]
    python -m mlx_batch_invariant_amd.dump_bits --compare bits_a.json bits_b.json

Counterpart of mlx-batch-invariant's harness/dump_bits.py:32-78. Determinism
is promised per (kernel library build, GPU, ROCm); this measures how far it
carries. Hashes (blake2b, 8 bytes, of the output's raw bytes) cover each op of
the reference's sweep (harness/sweep.py:65-179: matmul, addmm, 4-bit and
8-bit quantized matmul, RMSNorm, decode and causal prefill attention) on a
fixed probe input at batch 1, in fp16, bf16 and fp32, under the stock torch
path and under the batch-invariant mode; and, with --model, the row-0 logits
of a random-init Llama-shaped decoder in prefill and decode under both modes.
--compare prints, per section and mode, how many hashes agree and exits 1 if
an invariant-mode hash differs.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import platform
import sys
from pathlib import Path

import torch

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _h(t: torch.Tensor) -> str:
    return hashlib.blake2b(t.detach().contiguous().view(torch.uint8).cpu().numpy().tobytes(),
                           digest_size=8).hexdigest()


# Probe shapes: matmul / addmm / quantized matmul x[1, 4096] @ W[4096, 4096]^T,
# RMSNorm over 4096, decode attention 8 / 2 heads of 128 over 1000 keys,
# causal prefill 48 tokens against 300 keys.
K = N = 4096
HQ, HKV, DH = 8, 2, 128
L_DEC, TQ_PRE, L_PRE = 1000, 48, 300
QUANT = (("qmatmul_4b", 4, 64), ("qmatmul_8b", 8, 32))


def probe_inputs(dt: torch.dtype) -> dict:
    """Every probe input, on the CPU, drawn from one fixed generator (so a CPU
    checker can recompute the outputs from the same values)."""
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    rn = lambda *s: torch.randn(s, generator=g).to(dt)
    p = {"W": rn(N, K), "x": rn(1, K), "lin_b": rn(N)}
    for name, bits, gs in QUANT:
        wq, s, b = bi.quantize(p["W"].float(), group_size=gs, bits=bits, dtype=dt)
        p[name] = (wq.view(torch.int32), s, b)
    p["w_n"], p["x_n"] = rn(K), rn(1, K)
    p["q"], p["k"], p["v"] = rn(1, HQ, 1, DH), rn(1, HKV, L_DEC, DH), rn(1, HKV, L_DEC, DH)
    p["qp"], p["kp"], p["vp"] = rn(1, HQ, TQ_PRE, DH), rn(1, HKV, L_PRE, DH), rn(1, HKV, L_PRE, DH)
    return p


def _ops(dt: torch.dtype, dev: str):
    """(name, fn) pairs over probe_inputs(dt) moved to ``dev``."""
    from mlx_batch_invariant_amd import nn as bnn
    F = torch.nn.functional
    p = {k: (tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev)) for k, v in probe_inputs(dt).items()}
    x, W, lin_b = p["x"], p["W"], p["lin_b"]
    out = [("matmul", lambda: torch.matmul(x, W.t())),
           ("addmm", lambda: F.linear(x, W, lin_b))]
    for name, bits, gs in QUANT:
        wq, s, b = p[name]
        out.append((name, lambda wq=wq, s=s, b=b, bits=bits, gs=gs: bnn.quantized_matmul(
            x, wq, s, b, transpose=True, group_size=gs, bits=bits)))
    out.append(("rms_norm", lambda: F.rms_norm(p["x_n"], (K,), p["w_n"], 1e-5)))
    out.append(("sdpa_decode", lambda: F.scaled_dot_product_attention(p["q"], p["k"], p["v"], scale=DH ** -0.5,
                                                                       enable_gqa=True)))
    from torch.nn.attention.bias import causal_lower_right
    out.append(("sdpa_prefill", lambda: F.scaled_dot_product_attention(
        p["qp"], p["kp"], p["vp"], attn_mask=causal_lower_right(TQ_PRE, L_PRE), scale=DH ** -0.5, enable_gqa=True)))
    return out


def hash_array(t: torch.Tensor) -> str:
    """The dump's hash of a tensor's raw bytes (blake2b, 8 bytes)."""
    return _h(t)


def _library_hash() -> str | None:
    from mlx_batch_invariant_amd import _lib
    p = Path(_lib.__file__).with_name("libbi_kernels.so")
    return hashlib.blake2b(p.read_bytes(), digest_size=8).hexdigest() if p.exists() else None


def dump(model: str | None = None, dev: str = "cuda") -> dict:
    import mlx_batch_invariant_amd as bi
    props = torch.cuda.get_device_properties(0)
    out = {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None),
           "device": props.name, "arch": getattr(props, "gcnArchName", None), "library": _library_hash(),
           "os": platform.platform(), "ops": {}, "model": {}}
    for dt_name, dt in DTYPES.items():
        for op_name, fn in _ops(dt, dev):
            for inv in (False, True):
                with bi.set_batch_invariant_mode(enabled=inv, strict=inv):
                    y = fn()
                torch.cuda.synchronize()
                out["ops"][f"{op_name}/{dt_name}/{'inv' if inv else 'stock'}"] = _h(y)
    if model:
        name, _, layers = model.partition(":")
        if name != "llama":
            raise ValueError(f"unknown model {name!r} (supported: llama[:LAYERS])")
        from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
        for bits in (4, None):
            cfg = LlamaConfig(layers=int(layers or 2), bits=bits)
            m = LlamaShaped(cfg, device=dev, dtype=torch.bfloat16, seed=0)
            prompt = torch.randint(0, cfg.vocab, (1, 16), generator=torch.Generator().manual_seed(0)).to(dev)
            tag = f"llama{cfg.layers}-{'q4g64' if bits else 'bf16'}"
            for inv in (False, True):
                with bi.set_batch_invariant_mode(enabled=inv, strict=inv):
                    cache = m.new_cache(1, 17)
                    pre = m(prompt, cache, 0)
                    nxt = pre.argmax(-1, keepdim=True)
                    dec = m(nxt, cache, 16)
                torch.cuda.synchronize()
                mode = "inv" if inv else "stock"
                out["model"][f"{tag}/prefill/{mode}"] = _h(pre[0:1])
                out["model"][f"{tag}/decode/{mode}"] = _h(dec[0:1])
            del m
    return out


def _mode_of(key: str) -> str:
    """The mode a hash was taken in: the last path component ("inv" / "stock")."""
    return key.rsplit("/", 1)[-1]


def compare(a: dict, b: dict, file=sys.stdout) -> int:
    """Hash-by-hash comparison of two dumps.

    Prints each dump's platform line, then per section ("ops", "model") and
    mode how many of the entries both dumps hold agree, which disagree, and
    which appear in one dump only. Returns 1 when any invariant-mode entry
    disagrees (the property that must hold across builds, ROCm versions and
    machines); stock-mode differences are reported but not an error."""
    for label, d in (("A", a), ("B", b)):
        print(f"{label}: {d.get('device')} ({d.get('arch')}), torch {d.get('torch')}, HIP {d.get('hip')}, "
              f"library {d.get('library')}", file=file)
    status = 0
    for section in ("ops", "model"):
        ha, hb = a.get(section, {}), b.get(section, {})
        if not ha and not hb:
            continue
        tally: dict[str, tuple[int, list[str]]] = {}
        for key in sorted(ha.keys() & hb.keys()):
            n, bad = tally.get(_mode_of(key), (0, []))
            if ha[key] != hb[key]:
                bad = bad + [key]
            tally[_mode_of(key)] = (n + 1, bad)
        for mode, (n, bad) in sorted(tally.items()):
            print(f"[{section}] {mode}: {n - len(bad)} of {n} hashes agree", file=file)
            if bad:
                print(f"    differ: {', '.join(bad)}", file=file)
                if mode == "inv":
                    status = 1
        lonely = sorted(ha.keys() ^ hb.keys())
        if lonely:
            print(f"    in one dump only: {', '.join(lonely)}", file=file)
    print("invariant hashes " + ("DIFFER" if status else "agree"), file=file)
    return status


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--out")
    p.add_argument("--model", help="llama[:LAYERS] — a random-init Llama-3-8B-shape decoder (default 2 layers)")
    p.add_argument("--compare", nargs=2)
    a = p.parse_args(argv)
    if a.compare:
        return compare(json.loads(Path(a.compare[0]).read_text()), json.loads(Path(a.compare[1]).read_text()))
    if not a.out:
        p.error("--out or --compare is required")
    if not torch.cuda.is_available():
        print("dump_bits needs a GPU", file=sys.stderr)
        return 2
    d = dump(a.model)
    Path(a.out).write_text(json.dumps(d, indent=1))
    print(f"wrote {a.out}: {len(d['ops'])} op hashes, {len(d['model'])} model hashes")
    return 0


if __name__ == "__main__":
    sys.exit(main())
