"""CPU model of the fp8 KV cache format (OCP FP8 E4M3FN codes with one scale per cache).
TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker. The format has no counterpart in the
reference (its cache is bf16, python/qengine/engine.py:419); it is this build's F3 variant:

  code -> value   E4M3FN: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is
                  subnormal (m * 2^-9); S.1111.111 is NaN; no infinities; largest finite 448
  value -> code   x * inv_scale as an fp32 product (inv_scale = fp32(1 / scale)), saturated at
                  +-448, rounded to the nearest code with ties to even mantissa
  dequantize      code value * scale

The attention over an fp8 cache is checked by running the oracle's attention on the
dequantized cache (attn_oracle.attn_decode casts the cache to fp32). Pins are in
tests/test_kv8_oracle.py.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def _decode_table() -> np.ndarray:
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * m * 2.0 ** -9
        else:
            vals[c] = s * (1 + m / 8) * 2.0 ** (e - 7)
    return vals


DECODE = _decode_table()


def decode(codes) -> np.ndarray:
    """uint8 codes (any shape, or a torch uint8 / float8_e4m3fn tensor) -> float64 values."""
    if isinstance(codes, torch.Tensor):
        codes = codes.view(torch.uint8).cpu().numpy()
    return DECODE[np.asarray(codes, dtype=np.uint8)]


def inv_scale(scale: float) -> np.float32:
    return np.float32(1.0) / np.float32(scale)


def encode(x, scale: float) -> np.ndarray:
    """Values (float32 array-like) -> uint8 codes, as the prep kernel stores them."""
    y = np.asarray(x, dtype=np.float32) * inv_scale(scale)  # fp32 product
    y = y.astype(np.float64)
    out = np.empty(y.shape, dtype=np.uint8)
    nan = np.isnan(y)
    sign = np.signbit(y)
    a = np.minimum(np.abs(np.where(nan, 0.0, y)), E4M3_MAX)
    # quantum of the binade (2^-9 in the subnormal range), round half to even on the mantissa
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -9)))
    e = np.clip(e, -6, 8)
    quantum = 2.0 ** (e - 3)
    q = np.rint(a / quantum) * quantum  # numpy rint: ties to even
    q = np.minimum(q, E4M3_MAX)
    # value -> code through the positive half of the table
    pos_vals = DECODE[:0x7F]  # codes 0x00..0x7E (finite, non-negative)
    idx = np.searchsorted(pos_vals, q)
    code = idx.astype(np.uint8)
    code = np.where(sign & (q > 0), code | 0x80, code)
    code = np.where(sign & (q == 0), np.uint8(0x80), code)
    out[...] = np.where(nan, np.uint8(0x7F) | np.where(sign, np.uint8(0x80), np.uint8(0)), code)
    return out


def dequantize(codes, scale: float) -> torch.Tensor:
    """Codes -> float32 tensor of code * scale (the values the fp8 cache stands for)."""
    return torch.from_numpy((decode(codes) * float(scale)).astype(np.float32))
