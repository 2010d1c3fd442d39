"""Writes tests/golden/smoke_expected.npz: the eight correctness cases of the reference's
tests/smoke_test.cu (:486-493) with its exact inputs and expected outputs.

Inputs are the glibc ``rand()`` draws after ``srand(42)`` (smoke_test.cu:77-81, :438),
quantised to fp16 as the reference does before computing its CPU reference
(:125-138); the expected output is the reference's exact fp32 CPU attention
(``cpu_gqa_attention``, :35-74), restated in oracle/pkv_oracle.c.  The file stores, per
case, the shape, the CRC32 of the fp16 Q/K/V bytes (so tests can check they regenerate
the same inputs) and the expected fp32 output.

    make -C oracle && python tests/golden/make_smoke_fixtures.py
"""
import os
import sys
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import native  # noqa: E402


def main():
    data = {}
    for i in range(native.SMOKE_CASES):
        shape = native.smoke_case(i)
        q, k, v = native.smoke_inputs(i)
        q16, k16, v16 = q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)
        crc = zlib.crc32(q16.tobytes() + k16.tobytes() + v16.tobytes())
        out = native.cpu_gqa_attention(q16.astype(np.float32), k16.astype(np.float32),
                                       v16.astype(np.float32))
        data[f"shape_{i}"] = np.array(shape, dtype=np.int32)
        data[f"crc_{i}"] = np.array([crc], dtype=np.uint32)
        data[f"expected_{i}"] = out
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "smoke_expected.npz")
    np.savez_compressed(path, **data)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
