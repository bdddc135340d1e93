"""Writes fp8_e4m3_vectors.json: known answers for OCP FP8 E4M3 ("fn").

The expected values come from the format's definition (OCP 8-bit Floating
Point Specification v1.0, E4M3: bias 7, no infinities, S.1111.111 = NaN,
largest finite 448, subnormals m * 2^-9) written out here in plain Python,
independent of torch and of the oracle:

  decode[c]  value of each of the 256 codes;
  encode     hand-picked inputs with the code round-to-nearest-even gives,
             including every tie class, the subnormal/normal boundary, the
             top of the range (448, the 464 tie, the (464, 480) band that
             rounds into the NaN code like torch's cast), signed zeros,
             infinities and NaN.

Run: python tests/golden/make_fp8_vectors.py
"""

from __future__ import annotations

import json
import math
import struct
from pathlib import Path


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def value(code: int) -> float:
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    if e == 15 and m == 7:
        return math.nan
    v = m * 2.0**-9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -v if s else v


def main() -> None:
    decode = []
    for c in range(256):
        v = value(c)
        decode.append({"code": c, "f32_bits": None if math.isnan(v) else f32_bits(v), "nan": math.isnan(v)})

    # (input, expected code, why)
    cases = [
        (0.0, 0x00, "+0"),
        (-0.0, 0x80, "-0 keeps its sign"),
        (1.0, 0x38, "e=7 m=0"),
        (-1.0, 0xB8, "sign"),
        (1.125, 0x39, "exact m=1"),
        (1.0625, 0x38, "tie between 1 and 1.125 -> even (m=0)"),
        (1.1875, 0x3A, "tie between 1.125 and 1.25 -> even (m=2)"),
        (1.0625 + 2**-20, 0x39, "just above a tie rounds up"),
        (1.0625 - 2**-20, 0x38, "just below a tie rounds down"),
        (448.0, 0x7E, "largest finite"),
        (-448.0, 0xFE, "largest finite, negative"),
        (464.0, 0x7E, "tie between 448 and 480 -> even (m=6)"),
        (464.5, 0x7F, "above the tie rounds into the NaN code"),
        (479.0, 0x7F, "(464, 480) -> NaN code"),
        (480.0, 0x7F, ">= 480 -> NaN code"),
        (1.0e6, 0x7F, "large -> NaN code"),
        (-1.0e6, 0xFF, "large negative -> NaN code with sign"),
        (math.inf, 0x7F, "+inf -> NaN code"),
        (-math.inf, 0xFF, "-inf -> NaN code with sign"),
        (2.0**-6, 0x08, "smallest normal"),
        (2.0**-6 - 2.0**-10, 0x08, "tie between 7*2^-9 and 2^-6 -> even (code 8)"),
        (7 * 2.0**-9, 0x07, "largest subnormal"),
        (2.0**-9, 0x01, "smallest subnormal"),
        (2.0**-10, 0x00, "tie between 0 and 2^-9 -> even (0)"),
        (2.0**-10 + 2.0**-30, 0x01, "just above the first tie"),
        (3 * 2.0**-10, 0x02, "tie between 1 and 2 (x 2^-9) -> even (2)"),
        (5 * 2.0**-10, 0x02, "tie between 2 and 3 -> even (2)"),
        (-3 * 2.0**-10, 0x82, "negative subnormal tie"),
        (1e-45, 0x00, "fp32 denormal -> 0"),
        (-1e-45, 0x80, "negative fp32 denormal -> -0"),
        (0.3, 0x2A, "0.3 = 1.2 * 2^-2 -> m=1.6 -> rounds to m=2 (0.3125)"),
        (240.0, 0x77, "240 = 1.875 * 2^7"),
        (256.0, 0x78, "2^8"),
        (100.0, 0x6C, "100 = 1.5625 * 2^6 -> tie -> even m=4 (96)"),
    ]
    enc = [{"f32_bits": f32_bits(x), "code": c, "why": why} for x, c, why in cases]
    enc.append({"f32_bits": 0x7FC00000, "code": 0x7F, "why": "+NaN"})
    enc.append({"f32_bits": 0xFFC00000, "code": 0xFF, "why": "-NaN keeps its sign"})
    # self-check of the hand-written expectations against the value table:
    # every finite expected code must be a nearest code to its input.
    for item in enc:
        x = struct.unpack("<f", struct.pack("<I", item["f32_bits"]))[0]
        c = item["code"]
        if math.isnan(value(c)):
            assert math.isnan(x) or abs(x) > 464 or math.isinf(x), item
            continue
        best = min(abs(abs(x) - abs(value(k))) for k in range(127))
        assert abs(abs(x) - abs(value(c))) == best, item
    out = {"format": "OCP FP8 E4M3 (fn)", "decode": decode, "encode": enc}
    path = Path(__file__).with_name("fp8_e4m3_vectors.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()
