"""CPU pins for the fp8 KV format model (oracle/kv8_oracle.py): torch's own float8_e4m3fn
(an independent implementation of the OCP E4M3FN format) for decoding and for in-range rounding,
closed-form code values, saturation, ties to even, and round trips."""
import math

import numpy as np
import pytest
import torch

from oracle import kv8_oracle as K


def test_decode_table_equals_torch_float8_e4m3fn():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    t = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ours = K.decode(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(t), np.isnan(ours))
    assert np.array_equal(t[~np.isnan(t)], ours[~np.isnan(ours)])


def test_closed_form_codes():
    d = K.decode(np.array([0x38, 0x7E, 0x01, 0x08, 0x07, 0xFE, 0x40, 0x00, 0x80], dtype=np.uint8))
    assert list(d[:7]) == [1.0, 448.0, 2.0 ** -9, 2.0 ** -6, 7 * 2.0 ** -9, -448.0, 2.0]
    assert d[7] == 0.0 and d[8] == 0.0 and math.copysign(1, d[8]) < 0
    assert np.isnan(K.decode(np.array([0x7F, 0xFF], dtype=np.uint8))).all()


def test_encode_matches_torch_rounding_in_range():
    """Round to nearest even for |x| <= 448, as torch's cast to float8_e4m3fn."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-9, 6, 20000))).astype(np.float32)
    x = x[np.abs(x) <= 448]
    ours = K.encode(x, 1.0)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(K.decode(ours), K.decode(theirs))


def test_ties_go_to_even_and_values_saturate():
    vals = K.DECODE[:0x7F]
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    got = K.encode(mids, 1.0)
    lo = np.arange(0x7E, dtype=np.uint8)
    want = np.where(lo % 2 == 0, lo, lo + 1).astype(np.uint8)  # even mantissa code wins the tie
    assert np.array_equal(got, want)
    big = np.array([449.0, 464.0, 480.0, 1e30, np.inf, -1e30, -np.inf], dtype=np.float32)
    assert list(K.decode(K.encode(big, 1.0))) == [448.0] * 5 + [-448.0] * 2


@pytest.mark.parametrize("scale", [1.0, 0.5, 0.037, 3.0])
def test_round_trip_and_scale(scale):
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF, 0x80)], dtype=np.uint8)
    vals = (K.decode(codes) * scale).astype(np.float32)
    back = K.encode(vals, scale)
    if scale in (1.0, 0.5):  # exact products: every code comes back
        assert np.array_equal(back, codes)
    else:  # one fp32 rounding of v * (1/s) can move a value by at most one code
        assert np.abs(K.decode(back) - K.decode(codes)).max() <= np.abs(K.decode(codes)).max() * 2 ** -3
    deq = K.dequantize(codes, scale).numpy()
    assert np.allclose(deq, K.decode(codes) * scale, rtol=1e-7)


def test_a_dropped_rounding_is_detected():
    """Truncating instead of rounding (a plausible slip) fails the torch comparison."""
    x = np.array([1.1, 1.3, 3.7, 100.5], dtype=np.float32)
    trunc = np.floor(x / 2.0 ** (np.floor(np.log2(x)) - 3)) * 2.0 ** (np.floor(np.log2(x)) - 3)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert not np.array_equal(trunc, theirs)
    assert np.array_equal(K.decode(K.encode(x, 1.0)), theirs)
