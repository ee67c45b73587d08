"""Writes the known-answer vectors in tests/golden/ (run: python tests/golden/make_golden.py).

The reference (qengine) ships no golden vectors for its attention path, so these are computed
from the mathematics by the independent numpy models in tests/refmath.py, never by oracle/:
  prep   : RMSNorm1p in float64 with one bf16 rounding; RoPE with fp32 angles pos*inv_freq,
           cos/sin in float64 rounded to bf16, every elementwise op rounded to bf16.
  decode : softmax attention as explicit float64 loops (GQA head h reads KV head h // group),
           then bf16(bf16(o) * bf16(sigmoid(gate))).
Float64 evaluation differs from the reference's fp32 evaluation only where a value lies within
rounding noise of a bf16 rounding boundary, so consumers compare within 1-2 bf16 ulps and require
most elements to match exactly. Inputs are seeded numpy draws; bf16 arrays are stored as uint16
bit patterns.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from refmath import attention_fp64, bf16_bits, gated_output_model, rne_bf16, rope_model  # noqa: E402

D = 256


def bf16_from(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    return rne_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def prep_case(seed: int, hq: int, hkv: int, n: int, pos: int, max_len: int, theta: float, rd: int):
    rng = np.random.default_rng(seed)
    qg = bf16_from(rng, (n, hq * 2 * D), 3.0)
    k = bf16_from(rng, (n, hkv * D), 3.0)
    v = bf16_from(rng, (n, hkv * D))
    qnw = bf16_from(rng, (D,), 0.3)
    knw = bf16_from(rng, (D,), 0.3)
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, rd, 2, dtype=np.float32) / np.float32(rd)))).astype(np.float32)
    eps = 1e-6

    def norm(x, w):
        x64 = x.astype(np.float64)
        r = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
        return rne_bf16((x64 * r * (1.0 + w.astype(np.float64))).astype(np.float32))

    q_out = np.zeros((n, hq * D), np.float32)
    k_rows = np.zeros((n, hkv, D), np.float32)
    for t in range(n):
        ang = (np.float32(pos + t) * inv).astype(np.float64)
        cos = rne_bf16(np.cos(np.concatenate([ang, ang])).astype(np.float32))
        sin = rne_bf16(np.sin(np.concatenate([ang, ang])).astype(np.float32))
        qh = norm(qg[t].reshape(hq, 2 * D)[:, :D], qnw)
        kh = norm(k[t].reshape(hkv, D), knw)
        q_out[t] = rope_model(qh, cos, sin).reshape(-1)
        k_rows[t] = rope_model(kh, cos, sin)
    return dict(qg=bf16_bits(qg), k=bf16_bits(k), v=bf16_bits(v), qnw=bf16_bits(qnw),
                knw=bf16_bits(knw), inv_freq=inv, pos=np.int32(pos), max_len=np.int32(max_len),
                hq=np.int32(hq), hkv=np.int32(hkv), eps=np.float32(eps),
                q_out=bf16_bits(q_out), k_rows=bf16_bits(k_rows))


def decode_case(seed: int, hq: int, hkv: int, n: int, pos: int, max_len: int):
    rng = np.random.default_rng(seed)
    kc = bf16_from(rng, (hkv, max_len, D))
    vc = bf16_from(rng, (hkv, max_len, D))
    q = bf16_from(rng, (n, hq * D))
    qg = bf16_from(rng, (n, hq * 2 * D))
    out = np.zeros((n, hq * D), np.float32)
    for t in range(n):
        L = min(pos + t + 1, max_len)
        o64 = attention_fp64(q[t].reshape(hq, D), kc, vc, hq // hkv, L, D ** -0.5)
        gate = qg[t].reshape(hq, 2 * D)[:, D:].reshape(-1)
        out[t] = gated_output_model(o64.reshape(-1), gate)
    return dict(q=bf16_bits(q), qg=bf16_bits(qg), kc=bf16_bits(kc), vc=bf16_bits(vc),
                pos=np.int32(pos), hq=np.int32(hq), hkv=np.int32(hkv), out=bf16_bits(out))


CASES = {
    "prep_gqa6_rows3": lambda: prep_case(101, 24, 4, 3, 1021, 1024, 1e7, 64),   # pos+2 = 1023
    "prep_rows_past_cache": lambda: prep_case(102, 8, 2, 4, 62, 64, 1e7, 64),   # rows at 64, 65
    "prep_long_position": lambda: prep_case(103, 4, 1, 1, 131071, 131072, 1e7, 64),
    "decode_gqa6_rows2": lambda: decode_case(201, 24, 4, 2, 45, 48),
    "decode_gqa4_rows5_clamped": lambda: decode_case(202, 8, 2, 5, 30, 33),
    "decode_mha_row1": lambda: decode_case(203, 2, 2, 1, 0, 8),
}


def main():
    for name, make in CASES.items():
        np.savez_compressed(HERE / f"{name}.npz", **make())
        print("wrote", name)


if __name__ == "__main__":
    main()
