"""Seeded synthetic inputs for the attention tests (CPU tensors; tests move them to the GPU).

Shapes follow the reference: head_dim 256, per-q-head [q | gate] projection rows, KV cache
[Hkv, max_len, 256]. Norm weights are 0.3*N(0,1) as in the reference's unit test
(tests/test_kernels.py:311-312 of qengine). Cache rows are N(0,1) and taken as already normed
and roped.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

BF = torch.bfloat16
D = 256


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g: torch.Generator, *shape, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(*shape, generator=g) * scale).to(BF)


@dataclass
class DecodeCase:
    q: torch.Tensor      # [n, hq*D] bf16 (normed + roped query rows)
    qg: torch.Tensor     # [n, hq*2*D] bf16 (gate source)
    kc: torch.Tensor     # [hkv, max_len, D] bf16
    vc: torch.Tensor
    pos: int             # position of row 0
    hq: int
    hkv: int

    @property
    def n(self) -> int:
        return self.q.shape[0]


def decode_case(seed: int, hq: int, hkv: int, pos: int, n: int, max_len: int | None = None,
                fill: int | None = None, key_scale_frac: float = 0.0,
                key_scale: float = 8.0) -> DecodeCase:
    """Cache positions [0, fill) hold N(0,1) rows (default: every position the rows attend); the
    rest of the cache is zero. ``key_scale_frac`` of the filled key rows (seeded choice) are
    multiplied by ``key_scale`` to make sharp softmax peaks."""
    max_len = max_len if max_len is not None else pos + n
    fill = fill if fill is not None else min(pos + n, max_len)
    g = gen(seed)
    kc = torch.zeros(hkv, max_len, D, dtype=BF)
    vc = torch.zeros(hkv, max_len, D, dtype=BF)
    kc[:, :fill] = randn(g, hkv, fill, D)
    vc[:, :fill] = randn(g, hkv, fill, D)
    if key_scale_frac > 0:
        nsel = max(1, int(fill * key_scale_frac))
        idx = torch.randperm(fill, generator=g)[:nsel]
        kc[:, idx] = (kc[:, idx].float() * key_scale).to(BF)
    q = randn(g, n, hq * D)
    qg = randn(g, n, hq * 2 * D)
    return DecodeCase(q, qg, kc, vc, pos, hq, hkv)


@dataclass
class ProjRows:
    proj: torch.Tensor   # [n, width + pad] bf16, qg | k | v side by side (strided views below)
    hq: int
    hkv: int

    @property
    def qg(self):
        return self.proj[:, : self.hq * 2 * D]

    @property
    def k(self):
        a = self.hq * 2 * D
        return self.proj[:, a: a + self.hkv * D]

    @property
    def v(self):
        a = self.hq * 2 * D + self.hkv * D
        return self.proj[:, a: a + self.hkv * D]


def proj_rows(g: torch.Generator, n: int, hq: int, hkv: int, pad: int = 8) -> ProjRows:
    """Fused projection rows as the engine lays them out (qg | k | v) with a padded row stride,
    so qg/k/v are strided views. Scales follow the reference unit test: qg*3, k*3, v*1."""
    w = hq * 2 * D + 2 * hkv * D
    proj = torch.zeros(n, w + pad, dtype=BF)
    proj[:, : hq * 2 * D] = randn(g, n, hq * 2 * D, scale=3.0)
    proj[:, hq * 2 * D: hq * 2 * D + hkv * D] = randn(g, n, hkv * D, scale=3.0)
    proj[:, hq * 2 * D + hkv * D: w] = randn(g, n, hkv * D)
    return ProjRows(proj, hq, hkv)


def norm_weights(g: torch.Generator):
    return randn(g, D, scale=0.3), randn(g, D, scale=0.3)


def ulp_close(a: torch.Tensor, b: torch.Tensor, ulps: int = 1):
    """|a-b| <= ulps * bf16 spacing at max(|a|,|b|); NaN must match NaN. Returns (ok, max diff)."""
    a, b = a.float(), b.float()
    m = torch.maximum(a.abs(), b.abs())
    spacing = torch.where(m > 0, torch.exp2(torch.floor(torch.log2(m.clamp_min(1e-38))) - 7),
                          torch.full_like(m, 1e-38))
    both_nan = torch.isnan(a) & torch.isnan(b)
    ok = ((a - b).abs() <= ulps * spacing) | (a == b) | both_nan
    ok &= torch.isnan(a) == torch.isnan(b)
    return bool(ok.all()), (a - b).abs().nan_to_num().max().item()


def attn_close(out: torch.Tensor, ref: torch.Tensor):
    """The reference unit test's per-element bound |out-ref| <= 2^-6*|ref| + 2e-3
    (tests/test_kernels.py:353 of qengine) plus the BASELINE gate (max-abs <= 2e-2,
    mean-abs <= 2e-3). Returns (ok, max-abs, mean-abs)."""
    o, r = out.float(), ref.float()
    d = (o - r).abs()
    ok = bool((d <= 2.0 ** -6 * r.abs() + 2e-3).all())
    mx, mean = d.max().item(), d.mean().item()
    return ok and mx <= 2e-2 and mean <= 2e-3, mx, mean


def rope_close(a: torch.Tensor, ref: torch.Tensor, rd: int = 64, exact_frac: float = 0.999):
    """Prep outputs (q rows or cache rows, last dim a multiple of 256) against the oracle.
    Dims >= rd (not rotated): within 1 bf16 ulp. Rotated dims: within 2 ulps of the pair
    magnitude max(|y_c|, |y_partner|). A rotation keeps each pair's norm, while a 1-ulp flip of
    the normed input (fp32 summation order of the RMS) moves y by up to one ulp of the larger
    term, which is many ulps of y itself when the two rotated terms cancel. Also requires
    exact_frac of all elements to be bit-equal. Returns (ok, max diff, exact fraction)."""
    a = a.float().reshape(-1, D)
    r = ref.float().reshape(-1, D)
    half = rd // 2
    partner = torch.cat([r[:, half:rd], r[:, :half]], dim=1)
    mag = torch.cat([torch.maximum(r[:, :rd].abs(), partner.abs()), r[:, rd:].abs()], dim=1)
    mag = torch.maximum(mag, a.abs())
    spacing = torch.exp2(torch.floor(torch.log2(mag.clamp_min(1e-30))) - 7)
    ulps = torch.ones_like(spacing)
    ulps[:, :rd] = 2
    d = (a - r).abs()
    ok = bool((d <= ulps * spacing).all())
    frac = (a == r).float().mean().item()
    return ok and frac >= exact_frac, d.max().item(), frac
