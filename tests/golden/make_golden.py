"""Writes the golden fixtures in this directory.

The reference ships no test vectors for the Block-RVQ path, so these values
are derived by hand from the IEEE-754 definitions (binary16: 10 fraction bits;
bfloat16: 7 fraction bits; round to nearest, ties to even) and from reading
the reference's stage-selection rule (src/runtime.py:352-372).  Nothing here
runs the oracle or the library: every expected value is a literal whose
derivation is in the comment beside it.

reconstruct_golden.json: block_size 1, one row, codebook entry i is used by
column i; each case is W[0, i] = rne(rne(sum_s c_s[i]) * rne(s)).

route_golden.json: the scalar route-codebook weight of one (codebook_sum,
row_scale) pair in both of the reference's roundings:
  mode 0, PackedIDRouteLinear (src/runtime.py:89-97): the product in the
    buffers' dtype, then cast to x dtype: rne_x(rne_buf(cs * rs));
  mode 1, id_route_linear_matmul (src/triton_id_matmul.py:59-60): each
    operand cast to x dtype, product in x dtype: rne_x(rne_x(cs) * rne_x(rs)).
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

BF16 = {
    "1+2^-7": 0x3F81,       # bf16 1 + 2^-7 (fraction 1 of 7 bits)
    "1+2^-3": 0x3F90,       # 1 + 2^-3 (fraction 0x10)
}

# (name, buffer dtype, x dtype, codebook_sum bits, row_scale bits, mode 0 bits, mode 1 bits)
ROUTE = [
    ("bf16x_double_rounding", "f16", "bf16", 0x3C05, 0x3BFF, 0x3F80, 0x3F81),
    # cs = 1 + 2^-8 + 2^-10 (fp16 fraction 5), rs = 1 - 2^-11 (fp16 0x3BFF = 2^-1 * (2 - 2^-10)).
    # mode 0: cs*rs = 1 + 2^-8 + 2^-11 - 2^-19 - 2^-21, just below 1 + 2^-8 + 2^-11 (half an fp16 ulp
    #   2^-10 above 1 + 2^-8) -> fp16 1 + 2^-8 (0x3C04); that is a bf16 tie (half of 2^-7) whose even
    #   neighbour is 1.0 -> 0x3F80.
    # mode 1: rne_bf16(cs): 1 + 2^-8 + 2^-10 is above the tie -> 1 + 2^-7; rne_bf16(rs): 1 - 2^-11 is
    #   2^-11 from 1.0 and 2^-8 - 2^-11 from 1 - 2^-8 -> 1.0; product 1 + 2^-7 -> 0x3F81.
    ("f16x_double_rounding_bf16_buffers", "bf16", "f16", BF16["1+2^-7"], BF16["1+2^-3"], 0x3C88, 0x3C89),
    # cs*rs = (1 + 2^-7)(1 + 2^-3) = 1 + 2^-3 + 2^-7 + 2^-10.
    # mode 0: bf16 ulp 2^-7 in [1, 2): 2^-10 < half ulp -> 1 + 2^-3 + 2^-7, exact in fp16: fraction
    #   (2^-3 + 2^-7) * 1024 = 128 + 8 = 0x088 -> 0x3C88.
    # mode 1: both operands exact in fp16, product exact in fp16: fraction 128 + 8 + 1 = 0x089 -> 0x3C89.
    ("f16_tie_to_even", "f16", "f16", F16["-1.5"] & 0x7FFF, F16["1+2^-10"], 0x3E02, 0x3E02),
    # 1.5 * (1 + 2^-10) = 1.5 + 2^-10 + 2^-11: fp16 ulp 2^-10 at 1.5, remainder 2^-11 is a tie
    #   between fraction 0x201 (odd) and 0x202 (even) -> 0x3E02; both modes round the same product once.
    ("f16_negative_tie", "f16", "f16", F16["-1.5"], F16["1+2^-10"], 0xBE02, 0xBE02),
    # the same with the sign bit set.
    ("bf16x_fp16_product_overflow", "f16", "bf16", 0x7B53, 0x4000, 0x7F80, 0x47EA),
    # cs = 60000 (fp16 0x7B53: 2^15 * (1 + 851/1024)), rs = 2.
    # mode 0: the fp16 product 120000 exceeds 65504 -> +inf (0x7C00) -> bf16 +inf 0x7F80.
    # mode 1: rne_bf16(60000): 60000 / 2^15 = 1.8310546875 and 0.8310546875 * 128 = 106.375 -> fraction 106,
    #   1 + 106/128 = 1.828125, * 2^15 = 59904; * 2 = 119808 = 2^16 * 1.828125 -> exponent field
    #   127 + 16 = 143 = 0x8F, fraction 106 = 0x6A -> (0x8F << 7) | 0x6A = 0x47EA.
    ("bf16x_subnormal_tie", "f16", "bf16", 0x0003, F16["0.5"], 0x3400, 0x33C0),
    # cs = 3 * 2^-24 (fp16 subnormal 3), rs = 0.5: product 1.5 * 2^-24.
    # mode 0: fp16 subnormal unit 2^-24: 1.5 is a tie between 1 (odd) and 2 (even) -> 2 * 2^-24 = 2^-23,
    #   bf16 exponent field 127 - 23 = 104 = 0x68 -> 0x3400.
    # mode 1: 3 * 2^-24 and 0.5 are exact in bf16 and so is their product 1.5 * 2^-24: exponent field
    #   127 - 24 = 103 = 0x67, fraction 0.5 * 128 = 0x40 -> (0x67 << 7) | 0x40 = 0x33C0.
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
    route = [{"name": n, "buffer_dtype": b, "x_dtype": x, "codebook_sum_bits": c, "row_scale_bits": r,
              "mode0_bits": e0, "mode1_bits": e1} for n, b, x, c, r, e0, e1 in ROUTE]
    (HERE / "route_golden.json").write_text(json.dumps(route, indent=1) + "\n")
    (HERE / "active_stages.json").write_text(json.dumps(ACTIVE, indent=1) + "\n")


if __name__ == "__main__":
    main()
