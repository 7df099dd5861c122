"""Writes tests/golden/known_answers.json.

The values are TRANSCRIBED, not computed by the oracle: they come from the
reference's spec (w4a16 W4A16_SPEC.md:84-105 quantisation example, :146-171
packing example) and its tests (w4a16-kernel/tests/test_quant.py:34-47), plus
two hand-derived corner cases whose derivation is written next to them.
Run:  python tests/golden/make_known_answers.py
"""
from __future__ import annotations

import json
import os

CASES = [
    {   # W4A16_SPEC.md:148-165
        "name": "spec_pack_0xC2714F08", "kind": "pack", "K": 8, "N": 1,
        "codes": [8, 0, 15, 4, 1, 7, 2, 12], "words_u32": [0xC2714F08],
    },
    {   # test_quant.py:41-47: x[3,0] = 0xA -> 0xA << 12
        "name": "test_quant_nibble_position", "kind": "pack", "K": 8, "N": 1,
        "codes": [0, 0, 0, 0xA, 0, 0, 0, 0], "words_u32": [0xA << 12],
    },
    {   # test_quant.py:34-38: all fifteens -> every bit set
        "name": "test_quant_extreme_15", "kind": "pack", "K": 16, "N": 2,
        "codes": [15] * 32, "words_u32": [0xFFFFFFFF] * 4,
    },
    {   # W4A16_SPEC.md:84-105 (first group); zero = round(5.625) = 6, q = [8,0,15,4];
        # scale = 0.800048828125/15 in fp32 -> fp16 0x2AD4 (inputs are fp16);
        # second group [1,2,3,4]: scale 0.2, zero clamp(round(-5)) = 0,
        # q = clamp(round(W/0.2)) = [5, 10, 15, 15].
        "name": "spec_quant_example", "kind": "quantize", "K": 8, "N": 1, "G": 4,
        "W": [0.1, -0.3, 0.5, -0.1, 1.0, 2.0, 3.0, 4.0],
        "codes": [8, 0, 15, 4, 5, 10, 15, 15],
        "zeros_bits": [0x4600, 0x0000],
    },
    {   # hand-derived: scale = 0.9375/15 = 0.0625 (0x2C00); ties 0.5,1.5,2.5,7.5 go to
        # even; round(-0/0.0625) = -0.0 survives clamp -> zero bits 0x8000
        "name": "ties_and_negative_zero_point", "kind": "quantize", "K": 8, "N": 1, "G": 8,
        "W": [0, 0.03125, 0.09375, 0.15625, 0.9375, 0.5, 0.25, 0.46875],
        "codes": [0, 0, 2, 2, 15, 8, 4, 8],
        "zeros_bits": [0x8000], "scales_bits": [0x2C00],
    },
]


def main() -> None:
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(out, "w") as f:
        json.dump(CASES, f, indent=1)
    print("wrote", out)


if __name__ == "__main__":
    main()
