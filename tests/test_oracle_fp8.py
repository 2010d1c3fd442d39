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
import pytest
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


def test_e4m3_encode_round_trips_every_finite_code():
    finite = [c for c in range(256) if c not in (0x7F, 0xFF)]
    vals = oracle.E4M3_TABLE[finite]
    np.testing.assert_array_equal(oracle.quantize_e4m3(vals, 1.0), np.array(finite, dtype=np.uint8))


@pytest.mark.parametrize("scale", [1.0, 1.0 / 64, 0.37, 3.0])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_e4m3_encode_matches_torch_on_every_16_bit_input(dtype, scale):
    """Every fp16 / bf16 bit pattern (NaNs, infinities, subnormals, values past 448 after
    scaling) against torch's float8_e4m3fn cast of the clamped fp32 quotient."""
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
    theirs = (x.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    ours = oracle.quantize_e4m3(x.float().numpy(), scale)
    np.testing.assert_array_equal(ours, theirs.numpy())


def test_e4m3_encode_ties_and_boundaries():
    q = lambda v: int(oracle.quantize_e4m3(np.array([v], dtype=np.float32), 1.0)[0])
    assert q(2.0 ** -10) == 0x00            # half of the smallest subnormal: tie to even 0
    assert q(3 * 2.0 ** -10) == 0x02        # 1.5 subnormal steps: tie to even 2
    assert q(1.0 + 1.0 / 16) == 0x38        # halfway between 1 and 1.125: even mantissa 0
    assert q(1.0 + 3.0 / 16) == 0x3A        # halfway between 1.125 and 1.25: even mantissa 2
    assert q(464.0) == 0x7E and q(1e30) == 0x7E and q(-1e30) == 0xFE  # saturates at 448
    assert q(float("nan")) == 0x7F and q(-0.0) == 0x80


def test_append_kv_oracle_writes_only_the_tail_slots():
    gen = torch.Generator().manual_seed(3)
    k = torch.randn(6, 2, 4, 128, generator=gen)
    v = torch.randn(6, 2, 4, 128, generator=gen)
    table = torch.tensor([[5, 2, 0], [1, 3, 4], [0, 0, 0]], dtype=torch.int32)
    lens = torch.tensor([6, 12, 0], dtype=torch.int32)   # positions 5 (page 2, slot 1), 11, none
    kn, vn = torch.randn(3, 2, 128, generator=gen), torch.randn(3, 2, 128, generator=gen)
    k2, v2 = oracle.append_kv(k, v, table, lens, kn, vn)
    assert torch.equal(k2[2, :, 1], kn[0]) and torch.equal(v2[4, :, 3], vn[1])
    changed = (k2 != k).any(-1).nonzero().tolist()
    assert changed == [[2, 0, 1], [2, 1, 1], [4, 0, 3], [4, 1, 3]]


def test_planted_tie_rule_is_caught():
    """Rounding ties up instead of to the even code (a plausible encoder mistake) fails
    the comparison with torch that pins quantize_e4m3."""
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    a = np.minimum(np.abs(x.float().numpy()).astype(np.float64), 448.0)
    vals = oracle._E4M3_POS_VALUES
    hi = np.clip(np.searchsorted(vals, a), 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    ties_up = np.where(vals[hi] - a <= a - vals[lo], hi, lo).astype(np.uint8)
    finite = np.isfinite(x.float().numpy())
    theirs = (x.float().clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
              & 0x7F)
    assert (ties_up[finite] != theirs[finite]).any()
    assert (oracle.quantize_e4m3(x.float().numpy(), 1.0)[finite] & 0x7F == theirs[finite]).all()
