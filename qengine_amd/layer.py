"""Host-side mirror of the reference decode loop's gated-attention branch on the gfx950 ops.

The reference runs, per full-attention layer and pass of n rows (python/qengine/engine.py:448-458):
  pr  = fused projection rows [qg (Hq*2*256) | k (Hkv*256) | v (Hkv*256)]
  attn_prep(pr[:, :q0], pr[:, q0:k1], pr[:, k1:], q_norm, k_norm, inv_freq, pos, q, kc, vc, eps)
  attn_decode(q, kc, vc, pos, pr[:, :q0], part_o, part_ml, out)
with inv_freq built on the CPU in fp32 and moved (engine.py:409-410), per-layer kc/vc
[Hkv, max_len, 256] (engine.py:419) and a shared q / part_o / part_ml scratch (engine.py:405-408).
GatedAttention owns the same buffers and issues the same work, by default as the reference's two
calls; fused=True issues the fused attn_prep_decode instead (two launches instead of three,
bit-identical results; on gfx950 up to 0.7 us faster per layer-call for one row on caches up to
8k positions, up to 1.2 us slower for two rows and at 16k, where the fused kernel's single-slot
KV tile loop costs more than the launch it saves). It allocates only at construction, so a pass
can be captured in a hipGraph.
"""
from __future__ import annotations

import torch

from . import _C, alloc_partials, default_splits

HEAD_DIM = 256


def rope_inv_freq(theta: float, rotary_dim: int, device="cuda") -> torch.Tensor:
    """fp32 RoPE inverse frequencies, computed on the CPU and then moved, like the reference
    (engine.py:409-410)."""
    expo = torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim
    return (1.0 / (theta ** expo)).to(device)


class GatedAttention:
    """One gated full-attention layer's KV cache plus the decode-path calls for n <= n_max rows."""

    def __init__(self, hq: int, hkv: int, max_len: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                 rope_theta: float = 1e7, rotary_dim: int = 64, eps: float = 1e-6, n_max: int = 8,
                 splits: int | None = None, fused: bool = False, device="cuda"):
        d = HEAD_DIM
        self.hq, self.hkv, self.max_len, self.eps, self.fused = hq, hkv, max_len, eps, fused
        self.q_norm, self.k_norm = q_norm.to(device), k_norm.to(device)
        self.inv_freq = rope_inv_freq(rope_theta, rotary_dim, device)
        self.kc = torch.zeros(hkv, max_len, d, dtype=torch.bfloat16, device=device)
        self.vc = torch.zeros_like(self.kc)
        self.q = torch.zeros(n_max, hq * d, dtype=torch.bfloat16, device=device)
        self.splits = splits or default_splits(max_len, hkv)
        self.part_o, self.part_ml = alloc_partials(n_max, hq, self.splits, device)
        self.q0 = hq * 2 * d
        self.k1 = self.q0 + hkv * d
        self.width = self.k1 + hkv * d

    def __call__(self, proj: torch.Tensor, pos: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """proj: [n, >= width] bf16 projection rows (any row stride); pos: int32 device tensor,
        element 0 = position of row 0; out: [n, Hq*256] bf16 rows. Writes K/V of the n rows at
        pos..pos+n-1 and the gated attention output of each row into out."""
        n = proj.shape[0]
        pr = proj[:, : self.width]
        qg = pr[:, : self.q0]
        q = self.q[:n]
        prep = (qg, pr[:, self.q0: self.k1], pr[:, self.k1:], self.q_norm, self.k_norm,
                self.inv_freq, pos, q, self.kc, self.vc, self.eps)
        if self.fused:
            _C.attn_prep_decode(*prep, self.part_o, self.part_ml, out)
        else:
            _C.attn_prep(*prep)
            _C.attn_decode(q, self.kc, self.vc, pos, qg, self.part_o, self.part_ml, out)
        return out
