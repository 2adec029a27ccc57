"""Write tests/golden/quant_kat.json: hand-derived known answers of the MLX
affine packing (codes low-to-high inside uint32 words; reference
mlx_batch_invariant/kernels/quantized.py:1-8 and :59).

The words are written out by hand from the layout rule, not produced by the
code under test:
  4-bit, codes 1..8         -> 0x87654321 (code i in bits [4i, 4i+4))
  4-bit, codes 15,0,...,0   -> 0x0000000F
  4-bit, codes 0,...,0,15   -> 0xF0000000
  8-bit, codes 0x11..0x44   -> 0x44332211
  8-bit, codes 255,0,0,1    -> 0x010000FF
Run: python tests/golden/make_golden.py
"""

import json
from pathlib import Path

KAT = {
    "unpack": [
        {"bits": 4, "words": [0x87654321], "codes": [1, 2, 3, 4, 5, 6, 7, 8]},
        {"bits": 4, "words": [0x0000000F, 0xF0000000], "codes": [15, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 15]},
        {"bits": 4, "words": [0xFEDCBA98], "codes": [8, 9, 10, 11, 12, 13, 14, 15]},
        {"bits": 8, "words": [0x44332211], "codes": [0x11, 0x22, 0x33, 0x44]},
        {"bits": 8, "words": [0x010000FF, 0x80000000], "codes": [255, 0, 0, 1, 0, 0, 0, 128]},
    ],
}

if __name__ == "__main__":
    out = Path(__file__).resolve().parent / "quant_kat.json"
    out.write_text(json.dumps(KAT, indent=1) + "\n")
    print(f"wrote {out}")
