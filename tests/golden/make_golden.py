"""Writes tests/golden/kat_vectors.json: the known-answer vectors that the
reference's own tests hold for the affine decode/GEMV path, as data.

Sources (read as text; nothing from the reference is imported or run):
  * logan-qwen4/src/colisource.rs:996-1058  mlx_affine_decode_matches_lsb_first_mlx_packing
      literal packed words for 4/5/6/8-bit; two 32-column groups with
      (scale, bias) = (1, 0.5), (2, -1); expected code = (col % 32) & mask.
  * logan-qwen4/src/colisource.rs:1061-1079 mlx_affine_expert_aux_is_scale_then_bias
      aux = [scale 2.0][bias -1.0], group 64; expected (col % 16) * 2 - 1.
  * logan-qwen4/src/colisource.rs:1094-1123 dense_affine_adapter_maps_math_and_group_metadata
      5-bit, group 32, same expectations as the first case.
  * logan-qwen4/src/lib.rs:17056-17094  0x11 bytes (code 1), scale 1, bias 0, x = 1 -> y = 128
  * logan-qwen4/src/lib.rs:17015-17053  zero codes, scale 1, bias 1, x = 1 -> 128 (5-bit g128, 6-bit g64)
  * logan-spark/src/lib.rs:1327-1351    affine-8 code 2, scale 1, bias 0, I = 64 -> 128 (bf16 out)
  * logan-qwen4/src/lib.rs:17676-17694  MXFP4 canonical nibble order: bytes
      0x10 0x32 .. 0xfe with scale byte 127 hold 0, 0.5, 1, 1.5, 2, 3, 4, 6,
      -0, -0.5, .., -6 (element 2i in the low nibble).
  * logan-qwen4/src/lib.rs:17604-17651  MXFP4 projections: constant bytes
      0x22 / 0x44 / 0xaa / 0xcc (codes 2, 4, 10, 12: 1, 2, -1, -2), scale byte
      127 (1.0), I = 64, x = ((i % 7) - 3) / 8 -> value * sum(x).
  * logan-qwen4/src/lib.rs:17277-17348  stacked experts: expert 0 all-zero codes -> 0;
      expert 1 words 0x11111111 (code 1), scale 1, bias 0, x = 1, D = M = 64 ->
      64 * silu(64) * 64 per element (rel 1e-6).
The expected values below are the closed forms those tests assert.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

OUT = Path(__file__).resolve().parent / "kat_vectors.json"

DECODE_WORDS = {
    4: [0x76543210, 0xFEDCBA98, 0x76543210, 0xFEDCBA98],
    5: [0x8A418820, 0xC5A92839, 0xCA307B9A, 0x38BDAB49, 0xFFBBCDEB],
    6: [0x440C2040, 0xA2481C61, 0x3CE34C2C, 0x544D2450, 0xA6585D65, 0x7DE75C6D],
    8: [0x03020100, 0x07060504, 0x0B0A0908, 0x0F0E0D0C,
        0x13121110, 0x17161514, 0x1B1A1918, 0x1F1E1D1C],
}


def decode_case(bits: int) -> dict:
    words = DECODE_WORDS[bits] * 2  # second group repeats the packed codes
    mask = (1 << bits) - 1
    expected = []
    for col in range(64):
        code = (col % 32) & mask
        expected.append(code + 0.5 if col < 32 else code * 2.0 - 1.0)
    return {
        "source": "logan-qwen4/src/colisource.rs:996-1058",
        "bits": bits, "rows": 1, "cols": 64, "group_size": 32,
        "words": words, "scales": [1.0, 2.0], "biases": [0.5, -1.0],
        "expected": expected,
    }


def main() -> None:
    cases = [decode_case(b) for b in (4, 5, 6, 8)]
    cases.append({
        "source": "logan-qwen4/src/colisource.rs:1061-1079",
        "bits": 4, "rows": 1, "cols": 64, "group_size": 64,
        "words": [0x76543210, 0xFEDCBA98] * 4, "scales": [2.0], "biases": [-1.0],
        "expected": [(c % 16) * 2.0 - 1.0 for c in range(64)],
    })
    five = decode_case(5)
    five["source"] = "logan-qwen4/src/colisource.rs:1094-1123"
    cases.append(five)

    gemv = [
        {"source": "logan-qwen4/src/lib.rs:17056-17094", "bits": 4, "group_size": 64,
         "O": 3, "I": 128, "byte": 0x11, "scale": 1.0, "bias": 0.0, "x": 1.0,
         "expected": 128.0},
        {"source": "logan-qwen4/src/lib.rs:17015-17053", "bits": 5, "group_size": 128,
         "O": 2, "I": 128, "byte": 0x00, "scale": 1.0, "bias": 1.0, "x": 1.0,
         "expected": 128.0},
        {"source": "logan-qwen4/src/lib.rs:17015-17053", "bits": 6, "group_size": 64,
         "O": 3, "I": 128, "byte": 0x00, "scale": 1.0, "bias": 1.0, "x": 1.0,
         "expected": 128.0},
    ]
    spark = {"source": "logan-spark/src/lib.rs:1327-1351", "O": 2, "I": 64, "byte": 2,
             "scale": 1.0, "bias": 0.0, "x": 1.0, "expected": 128.0}
    silu64 = 64.0 / (1.0 + math.exp(-64.0))
    moe = {"source": "logan-qwen4/src/lib.rs:17277-17348", "bits": 4, "group_size": 64,
           "D": 64, "M": 64, "expert0_word": 0, "expert1_word": 0x11111111,
           "scale": 1.0, "bias": 0.0, "x": 1.0,
           "expected_expert0": 0.0, "expected_expert1": 64.0 * (silu64 * 64.0),
           "rel_tol": 1e-6}
    mx_order = {"source": "logan-qwen4/src/lib.rs:17676-17694",
                "bytes": [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], "scale_byte": 127,
                "expected": [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                             -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]}
    xs = [((i % 7) - 3.0) / 8.0 for i in range(64)]
    mx_proj = [{"source": "logan-qwen4/src/lib.rs:17604-17651", "O": o, "I": 64, "byte": b,
                "scale_byte": 127, "x": xs, "expected": v * sum(xs)}
               for o, b, v in ((64, 0x22, 1.0), (32, 0x44, 2.0), (32, 0xAA, -1.0),
                               (16, 0xCC, -2.0))]
    OUT.write_text(json.dumps({"decode": cases, "gemv": gemv, "spark_affine8": spark,
                               "expert": moe, "mxfp4_order": mx_order,
                               "mxfp4_gemv": mx_proj}, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
