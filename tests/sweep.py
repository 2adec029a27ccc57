"""Batch-sweep conformance protocol (reference: harness/sweep.py:36-40, :224-242).

A fixed probe row is embedded at the first and the last position of batches
of increasing size; its output must be bitwise identical to the batch-1 result.
Fillers are reseeded per (B, position) exactly like the reference harness.
"""

from __future__ import annotations

import torch

from helpers import bits, gen

DEFAULT_BATCHES = [1, 2, 3, 4, 8, 16, 32, 64, 128, 256]


def _cat(parts):
    if isinstance(parts[0], tuple):
        return tuple(torch.cat([p[i] for p in parts], 0) for i in range(len(parts[0])))
    return torch.cat(parts, 0)


def _slice(x, a, b):
    if isinstance(x, tuple):
        return tuple(t[a:b] for t in x)
    return x[a:b]


def sweep(probe, make_filler, run, batches=DEFAULT_BATCHES, seed=0, positions=None):
    """Return a list of (B, pos) whose probe output differs from batch 1."""
    ref = run(probe)
    ref_bits = bits(_slice(ref, 0, 1))
    fails = []
    for B in batches:
        pos_list = positions(B) if positions else sorted({0, B - 1})
        for pos in pos_list:
            g = gen(seed + 7 * B + pos)
            parts = []
            if pos > 0:
                parts.append(make_filler(pos, g))
            parts.append(probe)
            if B - 1 - pos > 0:
                parts.append(make_filler(B - 1 - pos, g))
            out = run(_cat(parts))
            if bits(_slice(out, pos, pos + 1)) != ref_bits:
                fails.append((B, pos))
    return fails
