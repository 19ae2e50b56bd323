"""Writes tests/golden/kat_int4.json: hand-derived known-answer vectors.

Every expected value below is written out literally and derived by hand from
the reference's definitions; none is computed by the oracle, so the oracle
(and the HIP kernels) are checked against them, not the other way round.

Derivations
-----------
pack_boundary      pare/tests/test_core.py:192-197 input [[0,15,0,15]].
                   byte = q[2b] | q[2b+1] << 4 (pare/core/pack.py:46-48)
                   -> [0 | 15<<4, 0 | 15<<4] = [0xF0, 0xF0].
pack_sequence      q = 1..8 -> bytes 0x21, 0x43, 0x65, 0x87.
repack_pattern     K = 32, group_size = 32, q[k] = k % 16. Kernel-layout byte j
                   (pare/core/pack.py:125-130) = q[j] | q[j+16] << 4 = j | j << 4
                   = 0x11 * j for j = 0..15. Storage bytes: q[2b] | q[2b+1] << 4
                   = (2b % 16) | ((2b+1) % 16) << 4.
scale_zero_asym    one group of 128 holding -0.5, 1.0 and otherwise values in
                   between. min = -0.5, max = 1.0 (pare/core/scale.py:85-86), so
                   scale = fp32(1.5 / 15) = fp32(0.1) and zero = round(0.5 / 0.1f)
                   = round(4.99999992..) where the fp32 quotient rounds to 5.0 -> 5.
                   q = clamp(round(x / scale + zero)) with fp32 division: x / 0.1f
                   for x in {0.25, 0.35, 0.05, 0.15, -0.45, 0.95} is exactly
                   {2.5, 3.5, 0.5, 1.5, -4.5, 9.5} after fp32 rounding, so
                   x/s + 5 = {7.5, 8.5, 5.5, 6.5, 0.5, 14.5} and round-half-even
                   gives {8, 8, 6, 6, 0, 14}; -0.5 -> 0, 1.0 -> 15, 0.0 -> 5.
scale_zero_pos     all values in [0.25, 4.0]: min clamps to 0 (scale.py:85),
                   scale = 4 / 15, zero = 0; 4.0 -> 15.
scale_zero_neg     all values in [-3.0, -1.5]: max clamps to 0 (scale.py:86),
                   scale = 3 / 15 = 0.2, zero = round(3 / 0.2f) = 15; -3.0 -> 0.
scale_zero_flat    all-zero group: scale clamps to 1e-8 (scale.py:88), zero = 0,
                   q = 0.
sym_unsigned_quirk sym=True on the unsigned grid (scale.py:73-82): scale =
                   absmax / 15 = 0.2 for absmax 3.0, zero = 0; every negative
                   value quantises to 0 (functional.py:70-74 clamps at qmin = 0).
dequant_pow2       (q - z) * s with s = 0.5, z = 8 (functional.py:91): q = 0 -> -4.0,
                   q = 15 -> 3.5, q = 8 -> 0.0, q = 3 -> -2.5; exact in fp32 and fp16.
dequant_f16_ties   scales s (given as fp32 bit patterns) and d = q - z for which
                   the fp32 product s * d is exactly half-way between two fp16
                   values while the exact product is not. The reference computes
                   the product in fp32 and then casts (linear.py:129), i.e. rounds
                   twice: "w16" is numpy's round-to-nearest-even fp16 of the fp32
                   product; "single" is the fp16 of the exact product (one
                   rounding), which a fused multiply-convert would produce
                   instead. Found by a seeded random search over s in
                   [0.001, 0.01]; listed literally.
"""

from __future__ import annotations

import json
from pathlib import Path

OUT = Path(__file__).resolve().parent / "kat_int4.json"


def main() -> None:
    asym_x = [-0.5, 1.0, 0.0, 0.25, 0.35, 0.05, 0.15, -0.45, 0.95]
    asym_q = [0, 15, 5, 8, 8, 6, 6, 0, 14]
    # pad the group to 128 with zeros (quantise to the zero point 5)
    asym_group = asym_x + [0.0] * (128 - len(asym_x))
    asym_q_full = asym_q + [5] * (128 - len(asym_q))

    kat = {
        "pack_boundary": {"q": [[0, 15, 0, 15]], "packed": [[0xF0, 0xF0]]},
        "pack_sequence": {"q": [[1, 2, 3, 4, 5, 6, 7, 8]], "packed": [[0x21, 0x43, 0x65, 0x87]]},
        "repack_pattern": {
            "group_size": 32,
            "q": [[k % 16 for k in range(32)]],
            "storage": [[(2 * b) % 16 | (((2 * b + 1) % 16) << 4) for b in range(16)]],
            "kernel": [[0x11 * j for j in range(16)]],
        },
        "scale_zero_asym": {"w": [asym_group], "group_size": 128, "scale": 0.1, "zero": 5.0,
                            "q": [asym_q_full]},
        "scale_zero_pos": {"w": [[0.25] * 127 + [4.0]], "group_size": 128,
                           "scale_num": 4.0, "scale_den": 15.0, "zero": 0.0,
                           "q_last": 15},
        "scale_zero_neg": {"w": [[-1.5] * 127 + [-3.0]], "group_size": 128,
                           "scale": 0.2, "zero": 15.0, "q_last": 0},
        "scale_zero_flat": {"w": [[0.0] * 128], "group_size": 128, "scale": 1e-8,
                            "zero": 0.0, "q": [[0] * 128]},
        "sym_unsigned_quirk": {"w": [[-3.0, -1.0, 0.0, 3.0] + [0.0] * 124], "group_size": 128,
                               "scale": 0.2, "zero": 0.0, "q_head": [0, 0, 0, 15]},
        "dequant_pow2": {"q": [[0, 15, 8, 3]], "scale": 0.5, "zero": 8.0,
                         "w": [[-4.0, 3.5, 0.0, -2.5]]},
        "dequant_f16_ties": [
            {"scale_bits": 994753468, "d": 15, "w16": 10736, "single": 10737},
            {"scale_bits": 995537211, "d": 13, "w16": 10612, "single": 10611},
            {"scale_bits": 1006722526, "d": 15, "w16": 12180, "single": 12181},
            {"scale_bits": 1007874867, "d": 5, "w16": 10686, "single": 10685},
            {"scale_bits": 1007874867, "d": 10, "w16": 11710, "single": 11709},
            {"scale_bits": 1008682780, "d": 9, "w16": 11674, "single": 11673},
        ],
    }
    OUT.write_text(json.dumps(kat, indent=1))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
