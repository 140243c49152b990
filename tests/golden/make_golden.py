"""Extract the reference's golden vectors into JSON fixtures.

Reads the numeric tables of tests/fp8_golden.h (PyTorch float8_e4m3fn -> FP32
bits for all 256 codes) and tests/rope_golden.h (Transformers v5.0.0 CPU FP32
YaRN cos/sin at positions 0, 1, 16383, 16384, 16385 and half-dims 1, 24, 40, 63)
from the reference checkout and writes only the numbers as data.

Usage: python tests/golden/make_golden.py [/root/reference]
"""
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def table(path, pattern):
    text = open(os.path.join(REF, path)).read()
    body = text[text.index("{"):]
    return [m for m in re.findall(pattern, body)]


def main():
    bits = [int(v, 16) for v in table("tests/fp8_golden.h", r"0x([0-9a-fA-F]+)u")]
    assert len(bits) == 256, len(bits)
    floats = [float(v) for v in table("tests/rope_golden.h",
                                      r"([-+]?\d\.\d+e[-+]\d+)f")]
    assert len(floats) == 5 * 4 * 2, len(floats)
    rope = [[[floats[(p * 4 + j) * 2], floats[(p * 4 + j) * 2 + 1]] for j in range(4)]
            for p in range(5)]
    with open(os.path.join(HERE, "fp8_golden.json"), "w") as f:
        json.dump({"source": "tests/fp8_golden.h",
                   "note": "FP32 bit patterns of float8_e4m3fn codes 0..255",
                   "bits": bits}, f, indent=0)
    with open(os.path.join(HERE, "rope_golden.json"), "w") as f:
        json.dump({"source": "tests/rope_golden.h",
                   "positions": [0, 1, 16383, 16384, 16385],
                   "half_dims": [1, 24, 40, 63],
                   "tolerance": 2e-6,
                   "cos_sin": rope}, f, indent=1)


if __name__ == "__main__":
    main()
