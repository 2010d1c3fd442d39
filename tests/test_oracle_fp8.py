"""Pins the oracle's e4m3 dequantisation (oracle/attention.py e4m3_value), which the fp8
K/V parity tests compare the engine against.

Checks: values fixed by the OCP FP8 E4M3 definition (zero, one, the largest normal 448,
the smallest normal 2^-6 and subnormal 2^-9, negative zero, the two NaN codes), the format's
monotone ordering of positive codes, and agreement with torch's independent
float8_e4m3fn conversion on all 256 codes.  A planted bias mistake (exponent bias 8, the
e4m3fnuz convention) is shown to fail the same checks.
"""
import math

import numpy as np
import torch

from oracle import attention as oracle


def test_e4m3_known_values():
    v = oracle.e4m3_value
    assert v(0x00) == 0.0 and math.copysign(1.0, v(0x80)) == -1.0
    assert v(0x38) == 1.0          # exponent 7, mantissa 0
    assert v(0x7E) == 448.0        # S.1111.110: the largest finite value
    assert v(0xFE) == -448.0
    assert v(0x08) == 2.0 ** -6    # smallest normal
    assert v(0x01) == 2.0 ** -9    # smallest subnormal
    assert v(0x07) == 7 * 2.0 ** -9
    assert math.isnan(v(0x7F)) and math.isnan(v(0xFF))
    assert sum(math.isnan(v(c)) for c in range(256)) == 2


def test_e4m3_positive_codes_are_monotone():
    pos = oracle.E4M3_TABLE[:0x7F]
    assert np.all(np.diff(pos) > 0)
    np.testing.assert_array_equal(oracle.E4M3_TABLE[0x80:0xFF], -pos[:0x7F])


def test_e4m3_matches_torch_float8_e4m3fn():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ours = oracle.dequantize_e4m3(codes, 1.0).numpy()
    theirs = codes.view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(ours), np.isnan(theirs))
    finite = ~np.isnan(ours)
    np.testing.assert_array_equal(ours[finite], theirs[finite])


def test_e4m3_scale_and_shape():
    x = torch.tensor([[0x38, 0xB8], [0x00, 0x7E]], dtype=torch.uint8)
    out = oracle.dequantize_e4m3(x, 0.5)
    assert out.shape == (2, 2) and out.dtype == torch.float32
    assert out.tolist() == [[0.5, -0.5], [0.0, 224.0]]


def test_bias_mistake_is_caught():
    """Decoding with bias 8 (the fnuz convention) halves every normal value."""
    wrong = np.array([0.0 if (c & 0x78) == 0 else
                      (-1.0 if c & 0x80 else 1.0) * 2.0 ** (((c >> 3) & 0xF) - 8) * (1 + (c & 7) / 8)
                      for c in range(256)], dtype=np.float32)
    assert wrong[0x38] != oracle.e4m3_value(0x38)
    assert not np.array_equal(wrong[:0x7F], oracle.E4M3_TABLE[:0x7F])
