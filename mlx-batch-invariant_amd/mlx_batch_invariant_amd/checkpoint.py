"""MLX-affine quantized checkpoints (safetensors) for torch models.

MLX (``mlx.nn.quantize`` / ``mlx_lm``) stores a quantized linear layer named
``<prefix>`` as three tensors, the format ``kernels/quantized.py:1-8`` of
mlx-batch-invariant describes and its kernels read directly:

* ``<prefix>.weight``  uint32 ``[N, K * bits / 32]``, codes packed low to high;
* ``<prefix>.scales``  ``[N, K / group_size]`` in the model dtype;
* ``<prefix>.biases``  ``[N, K / group_size]`` in the model dtype;

with the quantization parameters in the model directory's ``config.json``:
``{"quantization": {"group_size": 64, "bits": 4}}``, optionally overridden per
layer by ``config["quantization"][<prefix>] = {"group_size": ..., "bits": ...}``
(or ``false`` for a layer left unquantized). Weights may be split over several
``*.safetensors`` shards.

This module maps that format onto torch modules without converting it:
``load_into`` replaces every ``nn.Linear`` whose checkpoint entry is quantized
by a ``QuantizedLinear`` holding the packed words, scales and biases as they
are (the batch-invariant kernel consumes exactly those bytes), and copies
every other tensor into the matching parameter or buffer. ``save`` writes a
model back in the same layout, so a round trip is bit-exact.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Callable, Dict, Iterable, Optional

import torch

from .nn import QuantizedLinear

__all__ = ["read_tensors", "read_config", "quantization_for", "load_into", "load_dir", "save", "quantize_linears"]


def read_tensors(paths: Iterable[os.PathLike]) -> Dict[str, torch.Tensor]:
    """All tensors of the given safetensors files (shards may not repeat a key)."""
    from safetensors.torch import load_file
    out: Dict[str, torch.Tensor] = {}
    for p in paths:
        for k, v in load_file(str(p)).items():
            if k in out:
                raise ValueError(f"{k} appears in more than one shard")
            out[k] = v
    return out


def read_config(directory: os.PathLike) -> dict:
    p = Path(directory) / "config.json"
    return json.loads(p.read_text()) if p.exists() else {}


def quantization_for(config: dict, prefix: str) -> Optional[dict]:
    """The (group_size, bits) of layer `prefix`, or None if it is not quantized."""
    q = config.get("quantization") or config.get("quantization_config")
    if not q:
        return None
    per = q.get(prefix)
    if per is False:
        return None
    if isinstance(per, dict):
        return {"group_size": int(per["group_size"]), "bits": int(per["bits"])}
    return {"group_size": int(q.get("group_size", 64)), "bits": int(q.get("bits", 4))}


def _words_as_int32(w: torch.Tensor) -> torch.Tensor:
    """uint32 packed codes as int32 (the same bits; the kernels take either)."""
    if w.dtype == torch.int32:
        return w
    if w.dtype == torch.uint32:
        return w.view(torch.int32)
    raise TypeError(f"packed weight must be uint32, got {w.dtype}")


def _set_submodule(root: torch.nn.Module, name: str, module: torch.nn.Module) -> None:
    parent, _, leaf = name.rpartition(".")
    setattr(root.get_submodule(parent) if parent else root, leaf, module)


def _quantized_from_tensors(w, s, b, bias, group_size: int, bits: int) -> QuantizedLinear:
    wq = _words_as_int32(w)
    N, words = wq.shape
    K = words * 32 // bits
    if s.shape != (N, K // group_size) or b.shape != s.shape:
        raise ValueError(f"scales/biases {tuple(s.shape)}/{tuple(b.shape)} do not match weight {tuple(wq.shape)} "
                         f"at bits={bits}, group_size={group_size}")
    q = QuantizedLinear.__new__(QuantizedLinear)
    torch.nn.Module.__init__(q)
    q.in_features, q.out_features, q.group_size, q.bits = K, N, group_size, bits
    q.register_buffer("weight", wq.contiguous())
    q.register_buffer("scales", s.contiguous())
    q.register_buffer("biases", b.contiguous())
    q.bias = None if bias is None else torch.nn.Parameter(bias.contiguous())
    return q


def load_into(model: torch.nn.Module, tensors: Dict[str, torch.Tensor], config: Optional[dict] = None,
              key_map: Optional[Callable[[str], str]] = None, strict: bool = True) -> torch.nn.Module:
    """Load checkpoint `tensors` into `model` in place (returns it).

    Module / parameter names of the model are looked up in the checkpoint
    through `key_map` (identity by default). A layer with ``<name>.scales`` in
    the checkpoint becomes a ``QuantizedLinear`` on the model's device (an
    ``nn.Linear`` there is replaced; a ``QuantizedLinear`` takes the new bits);
    group size and bits come from `config` (``quantization_for``), else from
    the tensor shapes with the MLX defaults. With `strict`, every checkpoint
    tensor must be used and every model parameter / buffer filled."""
    config = config or {}
    km = key_map or (lambda k: k)
    used = set()
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, (torch.nn.Linear, QuantizedLinear)):
            continue
        key = km(name)
        if f"{key}.scales" not in tensors:
            continue
        q = quantization_for(config, key) or {}
        w = tensors[f"{key}.weight"]
        s = tensors[f"{key}.scales"]
        b = tensors.get(f"{key}.biases")
        if b is None:
            raise NotImplementedError(f"{key}: affine quantization needs biases (MLX mode 'affine')")
        bits = q.get("bits")
        if bits is None:
            K = getattr(mod, "in_features")
            bits = w.shape[1] * 32 // K
        gs = q.get("group_size") or (w.shape[1] * 32 // bits) // s.shape[1]
        ref = next(iter(mod.buffers()), None) if isinstance(mod, QuantizedLinear) else mod.weight
        device = ref.device if ref is not None and ref.device.type != "meta" else w.device
        bias = tensors.get(f"{key}.bias")
        new = _quantized_from_tensors(w.to(device), s.to(device), b.to(device),
                                      None if bias is None else bias.to(device), gs, bits)
        _set_submodule(model, name, new)
        used.update({f"{key}.weight", f"{key}.scales", f"{key}.biases"} | ({f"{key}.bias"} if bias is not None else set()))
    missing = []
    state = dict(model.named_parameters())
    state.update(dict(model.named_buffers()))
    for name, t in state.items():
        owner = name.rpartition(".")[0]
        if isinstance(model.get_submodule(owner) if owner else model, QuantizedLinear) and km(owner) + ".scales" in tensors:
            continue
        key = km(name)
        if key not in tensors:
            missing.append(name)
            continue
        src = tensors[key]
        if tuple(src.shape) != tuple(t.shape):
            raise ValueError(f"{name}: checkpoint shape {tuple(src.shape)} != model shape {tuple(t.shape)}")
        with torch.no_grad():
            t.copy_(src.to(device=t.device, dtype=t.dtype))
        used.add(key)
    if strict:
        unused = sorted(set(tensors) - used)
        if missing or unused:
            raise KeyError(f"checkpoint mismatch: missing {missing[:8]}{'...' if len(missing) > 8 else ''}, "
                           f"unused {unused[:8]}{'...' if len(unused) > 8 else ''}")
    return model


def load_dir(model: torch.nn.Module, directory: os.PathLike, key_map=None, strict: bool = True) -> torch.nn.Module:
    """``load_into`` with every ``*.safetensors`` shard and ``config.json`` of an
    MLX model directory."""
    d = Path(directory)
    shards = sorted(d.glob("*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"no *.safetensors in {d}")
    return load_into(model, read_tensors(shards), read_config(d), key_map=key_map, strict=strict)


def save(model: torch.nn.Module, directory: os.PathLike, key_map=None, config: Optional[dict] = None,
         shard_bytes: int = 4 << 30) -> None:
    """Write `model` as an MLX model directory: quantized layers as packed
    uint32 weight + scales + biases, everything else as is; ``config.json``
    gets the quantization parameters (a single default when every quantized
    layer shares them, per-layer entries otherwise)."""
    from safetensors.torch import save_file
    km = key_map or (lambda k: k)
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    tensors: Dict[str, torch.Tensor] = {}
    qparams: Dict[str, dict] = {}
    skip = set()
    for name, mod in model.named_modules():
        if isinstance(mod, QuantizedLinear):
            key = km(name)
            tensors[f"{key}.weight"] = mod.weight.detach().contiguous().view(torch.uint32).cpu()
            tensors[f"{key}.scales"] = mod.scales.detach().contiguous().cpu()
            tensors[f"{key}.biases"] = mod.biases.detach().contiguous().cpu()
            if mod.bias is not None:
                tensors[f"{key}.bias"] = mod.bias.detach().contiguous().cpu()
            qparams[key] = {"group_size": mod.group_size, "bits": mod.bits}
            skip.update({f"{name}.weight", f"{name}.scales", f"{name}.biases", f"{name}.bias"})
    for name, t in list(model.named_parameters()) + list(model.named_buffers()):
        if name in skip:
            continue
        tensors[km(name)] = t.detach().contiguous().cpu()
    # shard by size, keys in sorted order
    shards, cur, size = [], {}, 0
    for k in sorted(tensors):
        nb = tensors[k].numel() * tensors[k].element_size()
        if cur and size + nb > shard_bytes:
            shards.append(cur)
            cur, size = {}, 0
        cur[k] = tensors[k]
        size += nb
    if cur or not shards:
        shards.append(cur)
    n = len(shards)
    for i, sh in enumerate(shards):
        fname = "model.safetensors" if n == 1 else f"model-{i + 1:05d}-of-{n:05d}.safetensors"
        save_file(sh, str(d / fname), metadata={"format": "mlx"})
    cfg = dict(config or {})
    if qparams:
        distinct = {(v["group_size"], v["bits"]) for v in qparams.values()}
        if len(distinct) == 1:
            gs, bits = distinct.pop()
            cfg["quantization"] = {"group_size": gs, "bits": bits}
        else:
            first = next(iter(qparams.values()))
            cfg["quantization"] = {"group_size": first["group_size"], "bits": first["bits"], **qparams}
    (d / "config.json").write_text(json.dumps(cfg, indent=1))


def quantize_linears(model: torch.nn.Module, group_size: int = 64, bits: int = 4,
                     predicate: Optional[Callable[[str, torch.nn.Linear], bool]] = None) -> torch.nn.Module:
    """Replace every ``nn.Linear`` (for which `predicate(name, module)` holds)
    by a ``QuantizedLinear`` quantized from it, like ``mlx.nn.quantize``."""
    for name, mod in list(model.named_modules()):
        if isinstance(mod, torch.nn.Linear) and mod.in_features % group_size == 0 and (
                predicate is None or predicate(name, mod)):
            _set_submodule(model, name, QuantizedLinear.from_linear(mod, group_size=group_size, bits=bits))
    return model
