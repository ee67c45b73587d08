"""CPU restatement of qengine's gated-attention path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, as the checker or as the CPU baseline, never as the measured or shipped path.

Restates the reference op for op in torch on the CPU, with the same dtypes and bf16 rounding
points:
  * python/qengine/reference.py:132-136  rmsnorm1p
  * python/qengine/reference.py:158-176  rope_cos_sin, apply_rope
  * python/qengine/reference.py:252-272  attention_qkv_from_proj, attention_core
  * python/qengine/engine.py:409-410     inv_freq built on the CPU in fp32
  * csrc/attn.cu:1-2,35,52,78            n-row semantics: row t sits at position pos+t, writes the
                                         cache only below max_len, attends [0, min(pos+t+1, max_len))
Rounding chain (reference.py and csrc/attn.cu:40,46-48,146-148 agree):
  q, k   = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w))          one rounding
  rope   = bf16(bf16(x * c) + bf16(rot * s)), c, s = bf16(cos/sin(fp32 pos * inv_freq))
  out    = bf16(bf16(softmax(q.K * D^-0.5) . V) * bf16(sigmoid(gate)))   fp32 softmax and P.V

Parity pins for every function are in tests/test_oracle.py.
"""
from __future__ import annotations

import math

import numpy as np
import torch

BF16 = torch.bfloat16
F32 = torch.float32
HEAD_DIM = 256

__all__ = [
    "BF16", "F32", "HEAD_DIM", "rope_inv_freq", "rmsnorm1p", "rope_cos_sin", "apply_rope",
    "attention_qkv_from_proj", "attention_core", "attention_core_grouped", "attn_prep",
    "attn_decode", "attn_prefill", "flash_decode_fp64",
]


# ------------------------------------------------------------------------------------ prep math
def rope_inv_freq(theta: float, rd: int) -> torch.Tensor:
    """fp32 inverse frequencies for rotate-half RoPE over the first ``rd`` dims, built on the CPU
    as the reference builds them (engine.py:409-410, reference.py:163): theta^-(2i/rd)."""
    expo = torch.arange(0, rd, 2, dtype=F32) / rd
    return 1.0 / (theta ** expo)


def rmsnorm1p(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Zero-centred RMSNorm over the last dim, computed in fp32 and rounded once to x's dtype
    (reference.py:132-136)."""
    xf = x.to(F32)
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return ((xf * inv) * (1.0 + w.to(F32))).to(x.dtype)


def rope_cos_sin(pos: int, inv_freq: torch.Tensor, dtype=BF16):
    """cos/sin tables of length rd for one position: fp32 angles pos*inv_freq, evaluated in fp32,
    then cast to the activation dtype (reference.py:158-166)."""
    ang = torch.tensor(float(pos), dtype=F32) * inv_freq.to(F32)
    full = torch.cat([ang, ang])
    return full.cos().to(dtype), full.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE on the first rd dims of x (bf16, each elementwise op rounds); the
    remaining dims pass through unchanged (reference.py:169-176)."""
    rd = cos.shape[-1]
    head, tail = x[..., :rd], x[..., rd:]
    lo, hi = head[..., : rd // 2], head[..., rd // 2:]
    rotated = torch.cat([-hi, lo], dim=-1)
    return torch.cat([head * cos + rotated * sin, tail], dim=-1)


def attention_qkv_from_proj(qg_row, k_row, v_row, qnw, knw, pos: int, hq: int, hkv: int,
                            eps: float, inv_freq):
    """One projection row -> (q [hq, D] normed+roped, gate [hq*D], k [hkv, D] normed+roped,
    v [hkv, D]). Each q head's slice of qg is [q | gate] (reference.py:252-260)."""
    d = HEAD_DIM
    per_head = qg_row.reshape(hq, 2 * d)
    q, gate = per_head[:, :d], per_head[:, d:].reshape(-1)
    q = rmsnorm1p(q, qnw, eps)
    k = rmsnorm1p(k_row.reshape(hkv, d), knw, eps)
    v = v_row.reshape(hkv, d)
    cos, sin = rope_cos_sin(pos, inv_freq)
    return apply_rope(q, cos, sin), gate, apply_rope(k, cos, sin), v


# ---------------------------------------------------------------------------------- attention
def attention_core(q, gate, kc, vc, n: int) -> torch.Tensor:
    """Faithful restatement of reference.py:263-272: K/V repeated per GQA group in fp32, fp32
    scores and softmax over cache positions [0, n), P.V rounded to bf16, times bf16
    sigmoid(gate). q [hq, D] bf16, gate [hq*D] bf16, kc/vc [hkv, max_len, D] bf16.
    Materialises [hq, n, D] fp32 K and V (3.2 GB each at n = 128k): use
    ``attention_core_grouped`` for long caches."""
    hq, d = q.shape
    grp = hq // kc.shape[0]
    K = kc[:, :n].to(F32).repeat_interleave(grp, dim=0)
    V = vc[:, :n].to(F32).repeat_interleave(grp, dim=0)
    scores = torch.einsum("hd,hnd->hn", q.to(F32), K) * d ** -0.5
    probs = torch.softmax(scores, dim=-1)
    o = torch.einsum("hn,hnd->hd", probs, V).to(BF16).reshape(-1)
    return o * torch.sigmoid(gate)


def attention_core_grouped(q, gate, kc, vc, n: int) -> torch.Tensor:
    """Same mathematics as ``attention_core`` without the repeat: the ``grp`` q heads of one KV
    head are contracted against that head's fp32 K/V with a batched matmul. Differs from the
    faithful form only by fp32 summation order (pinned in tests/test_oracle.py)."""
    hq, d = q.shape
    hkv = kc.shape[0]
    grp = hq // hkv
    qh = q.to(F32).reshape(hkv, grp, d)
    K = kc[:, :n].to(F32)
    V = vc[:, :n].to(F32)
    scores = torch.bmm(qh, K.transpose(1, 2)) * d ** -0.5
    probs = torch.softmax(scores, dim=-1)
    o = torch.bmm(probs, V).to(BF16).reshape(-1)
    return o * torch.sigmoid(gate)


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(1, -1) if t.dim() == 1 else t


def attn_prep(qg, k, v, qnw, knw, inv_freq, pos: int, kc, vc, eps: float, hq: int):
    """n-row q/k prep + cache write with csrc/attn.cu:17-56 semantics, computed with the
    reference's row functions. Row t is at position pos+t; K/V are written only when
    pos+t < max_len (attn.cu:52). Mutates kc/vc in place and returns q_out [n, hq*D] bf16."""
    qg, k, v = _rows(qg), _rows(k), _rows(v)
    hkv, max_len, d = kc.shape
    n = qg.shape[0]
    q_out = torch.empty(n, hq * d, dtype=BF16)
    for t in range(n):
        p = pos + t
        q_r, _, k_r, v_r = attention_qkv_from_proj(qg[t], k[t], v[t], qnw, knw, p, hq, hkv, eps,
                                                   inv_freq)
        q_out[t] = q_r.reshape(-1)
        if p < max_len:
            kc[:, p] = k_r
            vc[:, p] = v_r
    return q_out


def attn_decode(q, kc, vc, pos: int, qg, hq: int, grouped: bool = True) -> torch.Tensor:
    """n-row gated attention with csrc/attn.cu:58-149 semantics: row t attends positions
    [0, min(pos+t+1, max_len)) with its gate taken from qg[t][h][D:2D] (attn.cu:147).
    Returns [n, hq*D] bf16."""
    q, qg = _rows(q), _rows(qg)
    hkv, max_len, d = kc.shape
    core = attention_core_grouped if grouped else attention_core
    out = torch.empty(q.shape[0], hq * d, dtype=BF16)
    for t in range(q.shape[0]):
        L = min(pos + t + 1, max_len)
        gate = qg[t].reshape(hq, 2 * d)[:, d:].reshape(-1)
        out[t] = core(q[t].reshape(hq, d), gate, kc, vc, L)
    return out


def attn_prefill(q, kc, vc, pos: int, qg, hq: int, row_block: int = 256) -> torch.Tensor:
    """Causal chunk: row t (position pos+t) attends [0, min(pos+t+1, max_len)). Mathematically
    ``attn_decode`` over all rows, evaluated with one fp32 batched matmul per block of rows and
    KV head (the reference has no prefill kernel; this is the per-row decode semantics of
    reference.py:263-272 applied to every row)."""
    q, qg = _rows(q), _rows(qg)
    hkv, max_len, d = kc.shape
    grp = hq // hkv
    T = q.shape[0]
    out = torch.empty(T, hq * d, dtype=BF16)
    gate_all = qg.reshape(T, hq, 2 * d)[:, :, d:].reshape(T, hq * d)
    for r0 in range(0, T, row_block):
        r1 = min(T, r0 + row_block)
        lens = torch.clamp(torch.arange(r0, r1) + pos + 1, max=max_len)
        Lmax = int(lens.max())
        K = kc[:, :Lmax].to(F32)
        V = vc[:, :Lmax].to(F32)
        Q = q[r0:r1].to(F32).reshape(r1 - r0, hkv, grp, d).permute(1, 0, 2, 3)
        Q = Q.reshape(hkv, (r1 - r0) * grp, d)
        scores = torch.bmm(Q, K.transpose(1, 2)) * d ** -0.5
        mask = torch.arange(Lmax)[None, :] >= lens[:, None]            # [rows, Lmax]
        mask = mask.repeat_interleave(grp, dim=0)[None]                 # [1, rows*grp, Lmax]
        scores = scores.masked_fill(mask, float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        o = torch.bmm(probs, V).reshape(hkv, r1 - r0, grp, d).permute(1, 0, 2, 3)
        o = o.reshape(r1 - r0, hq * d).to(BF16)
        out[r0:r1] = o * torch.sigmoid(gate_all[r0:r1])
    return out


# ------------------------------------------------------------------------- split-KV, in fp64
def flash_decode_fp64(q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float, bounds):
    """Flash-decoding restated in fp64 (csrc/attn.cu:58-149): each slice [b0, b1) of positions
    yields an unnormalised partial (o, m, l) by an online softmax; empty slices yield
    (0, -inf, 0) and are skipped by the log-sum-exp merge. Returns (merged output, partials).
    q [D], K/V [L, D]."""
    parts = []
    for b0, b1 in bounds:
        m, l, o = -math.inf, 0.0, np.zeros(K.shape[1])
        for p in range(b0, b1):
            s = float(q @ K[p]) * scale
            mn = max(m, s)
            corr = math.exp(m - mn) if m != -math.inf else 0.0
            e = math.exp(s - mn)
            o = o * corr + e * V[p]
            l = l * corr + e
            m = mn
        parts.append((o, m, l))
    M = max(p[1] for p in parts)
    L, O = 0.0, np.zeros(K.shape[1])
    for o, m, l in parts:
        if m == -math.inf:
            continue
        f = math.exp(m - M)
        L += l * f
        O += o * f
    return O / L, parts
