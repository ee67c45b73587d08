"""Independent numpy models used to pin the oracle: bf16 round-to-nearest-even done on the bit
pattern, and brute-force fp64 attention written as explicit loops. They share no code with
oracle/ (which is torch), so a mistake in one is not repeated in the other."""
from __future__ import annotations

import math

import numpy as np


def rne_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even) and return them as float32.
    NaN stays NaN; overflow rounds to inf as IEEE requires."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def bf16_bits(x) -> np.ndarray:
    """Upper 16 bits of float32 values that are exactly representable in bf16."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def rope_model(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE with every elementwise result rounded to bf16: the products of bf16
    values are exact in float64, so each step is one correctly rounded bf16 operation.
    x [..., D] (bf16 values as float32), cos/sin [rd] (bf16 values)."""
    rd = cos.shape[-1]
    half = rd // 2
    y = x.astype(np.float32).copy()
    x64 = x.astype(np.float64)
    c64, s64 = cos.astype(np.float64), sin.astype(np.float64)
    for i in range(rd):
        partner = -x64[..., i + half] if i < half else x64[..., i - half]
        a = rne_bf16((x64[..., i] * c64[i]).astype(np.float32))
        b = rne_bf16((partner * s64[i]).astype(np.float32))
        y[..., i] = rne_bf16((a.astype(np.float64) + b.astype(np.float64)).astype(np.float32))
    return y


def attention_fp64(q, K, V, grp: int, n: int, scale: float):
    """Brute-force softmax attention in float64 with explicit loops.
    q [hq, D]; K, V [hkv, >=n, D]; q head h reads KV head h // grp; positions [0, n)."""
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    hq, D = q.shape
    out = np.zeros((hq, D))
    for h in range(hq):
        kv = h // grp
        scores = [sum(q[h, d] * K[kv, p, d] for d in range(D)) * scale for p in range(n)]
        mx = max(scores)
        w = [math.exp(s - mx) for s in scores]
        tot = sum(w)
        for p in range(n):
            out[h] += (w[p] / tot) * V[kv, p]
    return out


def sigmoid64(x):
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-x))


def gated_output_model(o64: np.ndarray, gate_bf16: np.ndarray) -> np.ndarray:
    """bf16(bf16(o) * bf16(sigmoid(gate))): the reference's epilogue rounding points, with o and
    sigmoid evaluated in float64 (the reference evaluates them in fp32)."""
    o = rne_bf16(o64.astype(np.float32)).astype(np.float64)
    s = rne_bf16(sigmoid64(gate_bf16).astype(np.float32)).astype(np.float64)
    return rne_bf16((o * s).astype(np.float32))
