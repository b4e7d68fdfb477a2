"""Writes reference_kats.json: the known-answer vectors of the reference's own
unit tests, as data (inputs and expected outputs).

  q4_0_dequant_0x88   crates/gguf/src/dequant.rs:235-252
  q8_0_dequant_2s     crates/gguf/src/dequant.rs:254-270
  q8_gemv_identity    crates/engine/src/q8_gemv.rs:257-281
The patterned parallel-vs-scalar GEMV test (q8_gemv.rs:283-314) is generated
in tests/test_oracle.py from its closed-form pattern.
Run: python tests/golden/make_reference_kats.py
"""
import json
import os

import numpy as np


def f16_le(v):
    b = int(np.array([v], np.float16).view(np.uint16)[0])
    return [b & 0xFF, b >> 8]


def main():
    kats = {}
    kats["q4_0_dequant_0x88"] = {"block": f16_le(1.0) + [0x88] * 16, "expected": [0.0] * 32}
    kats["q8_0_dequant_2s"] = {"block": f16_le(0.5) + [2] * 32, "expected": [1.0] * 32}
    m, n = 4, 32
    w = []
    for row in range(m):
        blk = f16_le(1.0) + [0] * 32
        blk[2 + row] = 1
        w += blk
    kats["q8_gemv_identity"] = {"m": m, "n": n, "w": w, "x": [float(i) for i in range(32)],
                                "expected": [float(i) for i in range(m)]}
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(out, "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
