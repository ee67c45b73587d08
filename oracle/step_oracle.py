"""CPU restatement of the rest of qengine's decode step around the attention path: embedding
gather, RMSNorm1p with the fused residual add, SwiGLU, argmax, and the device-side step
bookkeeping (accept / commit / mtp_select). TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker; it is never the measured or shipped path.

  embed(table, tok, n)            csrc/basic.cu:16-26   (ids outside the table give zero rows)
  residual_rmsnorm1p(h, d, w, eps) csrc/basic.cu:34-54, python/qengine/reference.py:132-136
                                  (h = bf16(h + d) first, then the oracle's rmsnorm1p)
  swiglu(gu)                      python/qengine/reference.py:283-287 (silu and the product each
                                  round to bf16), csrc/basic.cu:160-170
  argmax(x)                       torch.argmax semantics (csrc/basic.cu:176-239): NaN is the
                                  maximum, ties go to the lowest index
  accept / commit / mtp_select    csrc/basic.cu:241-307, on plain Python lists of ints

Parity pins are in tests/test_step_oracle.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .attn_oracle import rmsnorm1p

BF16 = torch.bfloat16


def embed(table: torch.Tensor, tok, n: int) -> torch.Tensor:
    V, H = table.shape
    out = torch.zeros(n, H, dtype=table.dtype)
    for r in range(n):
        t = int(tok[r])
        if 0 <= t < V:
            out[r] = table[t]
    return out


def residual_rmsnorm1p(h: torch.Tensor, d: torch.Tensor | None, w: torch.Tensor, eps: float):
    """Returns (new residual stream, normalised rows)."""
    if d is not None:
        h = (h + d)  # a bf16 torch add: one rounding
    return h, rmsnorm1p(h, w, eps)


def swiglu(gu: torch.Tensor) -> torch.Tensor:
    I = gu.shape[-1] // 2
    return F.silu(gu[..., :I]) * gu[..., I:]


def argmax(x: torch.Tensor) -> torch.Tensor:
    """Per row: the first NaN if there is one, else the first index of the maximum."""
    xs = x.float().reshape(-1, x.shape[-1])
    out = []
    for row in xs:
        nan = torch.isnan(row).nonzero()
        if len(nan):
            out.append(int(nan[0]))
        else:
            out.append(int((row == row.max()).nonzero()[0]))
    return torch.tensor(out, dtype=torch.int32)


def accept(in_tok: list, am: list, n: int, ctl: list, next_tok: list, log: list) -> None:
    """In place on lists, like the device kernel on int32 buffers."""
    P, mode, max_len = ctl[0], ctl[2], len(log)
    m = n - 1
    if mode == 1:
        m = 0
        while m < n - 1 and in_tok[m + 1] == am[m]:
            m += 1
        for i in range(m + 1):
            if 0 <= P + 1 + i < max_len:
                log[P + 1 + i] = am[i]
        ctl[4] += 1
        ctl[5] += m
        ctl[16 + m] += 1
    elif in_tok[n] < 0 and 0 <= P + n < max_len:
        log[P + n] = am[n - 1]
    for r in range(n):
        if mode == 1:
            next_tok[r] = am[r]
        elif r + 1 < n:
            next_tok[r] = in_tok[r + 1]
        else:
            next_tok[r] = in_tok[n] if in_tok[n] >= 0 else am[n - 1]
    ctl[3] = m


def commit(ctl: list, in_tok: list, am: list, drafts: list, k: int) -> None:
    m = ctl[3]
    ctl[0] += m + 1
    ctl[1] = m + 1
    in_tok[0] = am[m]
    for j in range(k):
        in_tok[1 + j] = drafts[j]


def mtp_select(ctl: list, off: int, src: torch.Tensor | None = None, mtp_am: list | None = None):
    """Returns (mpos, selected src row or None, draft0 or None)."""
    m = ctl[3]
    mpos = ctl[0] if off < 0 else ctl[0] + m + 1 + off
    row = src[m].clone() if src is not None else None
    d0 = mtp_am[m] if mtp_am is not None else None
    return mpos, row, d0
