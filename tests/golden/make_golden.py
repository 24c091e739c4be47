"""Writes the golden fixtures in this directory.

The reference ships no test vectors for the Block-RVQ path, so these values
are derived by hand from the IEEE-754 definitions (binary16: 10 fraction bits;
bfloat16: 7 fraction bits; round to nearest, ties to even) and from reading
the reference's stage-selection rule (src/runtime.py:352-372).  Nothing here
runs the oracle or the library: every expected value is a literal whose
derivation is in the comment beside it.

reconstruct_golden.json: block_size 1, one row, codebook entry i is used by
column i; each case is W[0, i] = rne(rne(sum_s c_s[i]) * rne(s)).
"""
from __future__ import annotations

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent

# fp16 bit patterns used below
F16 = {
    "1": 0x3C00,            # 1.0
    "1+2^-10": 0x3C01,      # 1 + 1 ulp(fp16)
    "1+2^-8": 0x3C04,       # 1 + 2^-8 (a bf16 tie point)
    "1+3*2^-8": 0x3C0C,     # 1 + 2^-7 + 2^-8 (a bf16 tie point)
    "1+2^-7": 0x3C08,
    "2^-24": 0x0001,        # smallest fp16 subnormal
    "-1.5": 0xBE00,
    "0.5": 0x3800,
    "2^-9": 0x1800,         # 2^-9
    "2^-8+2^-11": 0x1C80,   # 2^-8 * (1 + 2^-3): exponent -8 -> field 7 (0x1C00), fraction 0.125*1024 = 0x080
    "-0": 0x8000,
}

CASES = [
    {
        "name": "s1_bf16_ties_and_subnormal",
        "out_dtype": "bf16",
        "stages": [[F16["1"], F16["1+2^-10"], F16["1+2^-8"], F16["1+3*2^-8"], F16["2^-24"], F16["-1.5"]]],
        "row_scale": F16["1"],
        "expected": [
            0x3F80,  # 1.0
            0x3F80,  # 1 + 2^-10 is below half a bf16 ulp (2^-8): rounds to 1.0
            0x3F80,  # 1 + 2^-8 is a tie; the even neighbour is 1.0
            0x3F82,  # 1 + 2^-7 + 2^-8 is a tie between 1+2^-7 (odd) and 1+2^-6 (even)
            0x3380,  # 2^-24: exponent field 127 - 24 = 103 = 0x67, fraction 0
            0xBFC0,  # -1.5: sign, exponent 127, fraction 0x40
        ],
    },
    {
        "name": "s1_bf16_product_rounding",
        "out_dtype": "bf16",
        "stages": [[F16["1+2^-7"], F16["-1.5"]]],
        "row_scale": F16["1+2^-7"],
        "expected": [
            0x3F82,  # (1+2^-7)^2 = 1 + 2^-6 + 2^-14 -> 1 + 2^-6 (remainder < half ulp)
            0xBFC2,  # -1.5 * (1+2^-7) = -(1.5 + 1.5*2^-7) = -1.5*(1 + 2^-7): fraction 0x40 + 0x01.8 -> tie? 1.5*2^-7 = 2^-7 + 2^-8:
                     # -1.5 - 2^-7 - 2^-8 ; bf16 ulp at 1.5 is 2^-7 -> -1.5 - 2^-7 - 2^-8 is a tie between
                     # -(1.5 + 2^-7) (fraction 0x41, odd) and -(1.5 + 2^-6) (fraction 0x42, even) -> 0xBFC2
        ],
    },
    {
        "name": "s2_bf16_sum_then_round",
        "out_dtype": "bf16",
        "stages": [[F16["1"], F16["1"], F16["-0"]], [F16["2^-9"], F16["2^-8+2^-11"], F16["-0"]]],
        "row_scale": F16["1"],
        "expected": [
            0x3F80,  # 1 + 2^-9: below half ulp -> 1.0
            0x3F81,  # 1 + 2^-8 + 2^-11: above the tie -> 1 + 2^-7
            0x0000,  # (0 + -0) + -0 = +0 in fp32 (the sum starts from +0), times 1 -> +0
        ],
    },
    {
        "name": "s1_f16_product_rounding",
        "out_dtype": "f16",
        "stages": [[F16["1+2^-10"], F16["-1.5"], F16["2^-24"]]],
        "row_scale": F16["1+2^-10"],
        "expected": [
            0x3C02,  # (1+2^-10)^2 = 1 + 2^-9 + 2^-20 -> 1 + 2^-9 (fraction 2)
            0xBE02,  # -1.5*(1+2^-10) = -(1.5 + 1.5*2^-10): fp16 ulp at 1.5 is 2^-10; 1.5*2^-10 = 2^-10 + 2^-11
                     # -> tie between fraction 0x201 (odd) and 0x202 (even) -> 0xBE02
            0x0001,  # 2^-24 * (1+2^-10) = 2^-24 + 2^-34 -> 2^-24 (subnormal unit)
        ],
    },
    {
        "name": "s1_f16_scale_half",
        "out_dtype": "f16",
        "stages": [[F16["-1.5"], F16["2^-24"]]],
        "row_scale": F16["0.5"],
        "expected": [
            0xBA00,  # -0.75: exponent 14, fraction 0x200
            0x0000,  # 2^-25 is a tie between 0 (even) and 2^-24 (odd) -> +0
        ],
    },
]

ACTIVE = [
    {"stages_per_split": [3], "effective": 3, "expected": [0, 1, 2]},
    {"stages_per_split": [3], "effective": 1, "expected": [0]},
    {"stages_per_split": [3], "effective": 0, "expected": [0]},     # keep = max(1, k)
    {"stages_per_split": [3], "effective": 5, "expected": [0, 1, 2]},
    {"stages_per_split": [3, 3, 3, 3], "effective": 2, "expected": [0, 1, 3, 4, 6, 7, 9, 10]},  # split-major
    {"stages_per_split": [2, 1], "effective": 2, "expected": [0, 1, 2]},
    {"stages_per_split": [1, 3], "effective": 2, "expected": [0, 1, 2]},
    {"stages_per_split": [], "effective": 1, "expected": [0]},        # empty -> [0]
]


def main() -> None:
    out = []
    for c in CASES:
        n = len(c["stages"][0])
        out.append({
            "name": c["name"],
            "out_dtype": c["out_dtype"],
            "d": 1,
            "K": n,
            "in_features": n,
            "ids": [list(range(n)) for _ in c["stages"]],
            "codebook_bits": [[v - 0x10000 if v >= 0x8000 else v for v in st] for st in c["stages"]],
            "row_scale_bits": c["row_scale"] - 0x10000 if c["row_scale"] >= 0x8000 else c["row_scale"],
            "expected_bits": c["expected"],
        })
    (HERE / "reconstruct_golden.json").write_text(json.dumps(out, indent=1) + "\n")
    (HERE / "active_stages.json").write_text(json.dumps(ACTIVE, indent=1) + "\n")


if __name__ == "__main__":
    main()
