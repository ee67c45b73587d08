"""CPU restatement of qengine's Gated DeltaNet decode/verify step with lazy rollback.
TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker; it is never the measured or shipped path.

Math per token (python/qengine/reference.py:211-242, which mirrors HF's qwen3_5
causal_conv1d_update / torch_recurrent_gated_delta_rule / RMSNormGated), per value head j with
qk head j // (Hv/Hk) (repeat_interleave, reference.py:225-229):
  conv    y_c = bf16(sum_w w[c][w] * [x_{t-3}, x_{t-2}, x_{t-1}, x_t][w]) in fp32, then
          bf16(silu(y_c))                                              reference.py:215-220
  gates   beta = bf16(sigmoid(b_j)); decay = exp(-exp(A_log_j) * softplus(a_j + dt_bias_j)),
          softplus with threshold 20                                   reference.py:224
  q, k    q = l2norm(q) / sqrt(128), k = l2norm(k) in fp32, l2norm(x) = x * rsqrt(|x|^2 + 1e-6)
  state   S = decay S; kv = S^T k; delta = beta (v - kv); S += k delta^T; o = bf16(S^T q)
                                                                       reference.py:234-239
  output  bf16(bf16(w * bf16(o * rsqrt(mean(o^2) + eps))) * silu(z))   reference.py:139-146

Pass semantics of the device kernel (csrc/gdn.cu:1-25, 85-131), which this module models on
plain tensors:
  * the committed state S is the state after position pos - pending; a pass first replays the
    ``pending`` rows the previous pass staged (k, v, decay, beta) into S and writes S back;
  * its n new rows (positions pos .. pos+n-1) run from a copy of S, are staged for the next pass,
    and S itself is not advanced by them;
  * the conv history is a ring of 16 slots keyed by absolute position (slot = position & 15),
    holding raw qkv rows; a row reads positions < pos from the ring (positions < 0 read as 0)
    and earlier rows of the same pass from the pass's own inputs; the pass writes its rows' slots.
The engine then sets pos += keep, pending = keep (tests/test_kernels.py:194-195 of the reference).

Parity pins are in tests/test_gdn_oracle.py.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32
DK = DV = 128
RING = 16
MAXN = 8


def conv_dim(hk: int, hv: int) -> int:
    return 2 * hk * DK + hv * DV


def conv_silu(hist: torch.Tensor, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """hist [C, 3] bf16 (x at t-3, t-2, t-1), x [C] bf16, w [C, 4] bf16 -> [C] bf16."""
    buf = torch.cat([hist, x[:, None]], dim=-1)
    conv = (buf.float() * w.float()).sum(-1).to(BF16)  # fp32 accumulate, one rounding
    return F.silu(conv)  # bf16 in, bf16 out


def gates(b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """b, a [Hv] bf16 -> (decay [Hv] fp32, beta [Hv] fp32 holding bf16 values)."""
    beta = b.sigmoid().float()
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    return g.exp(), beta


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def split_heads(y: torch.Tensor, hk: int, hv: int):
    """Conv output [C] -> q [Hv, 128] (scaled), k [Hv, 128], v [Hv, 128], all fp32."""
    r = hv // hk
    q = y[: hk * DK].view(hk, DK).repeat_interleave(r, dim=0)
    k = y[hk * DK: 2 * hk * DK].view(hk, DK).repeat_interleave(r, dim=0)
    v = y[2 * hk * DK:].view(hv, DV)
    return l2norm(q.float()) / math.sqrt(DK), l2norm(k.float()), v.float()


def delta_update(S: torch.Tensor, k: torch.Tensor, v: torch.Tensor, decay: torch.Tensor,
                 beta: torch.Tensor) -> None:
    """S [Hv, 128, 128] fp32 in place; k, v [Hv, 128]; decay, beta [Hv]."""
    S.mul_(decay[:, None, None])
    kv = (S * k[:, :, None]).sum(dim=1)
    delta = (v - kv) * beta[:, None]
    S.add_(k[:, :, None] * delta[:, None, :])


def read_out(S: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    return (S * q[:, :, None]).sum(dim=1).to(BF16)  # [Hv, 128]


def gated_rmsnorm(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """o, z [Hv, 128] bf16, w [128] bf16 -> [Hv, 128] bf16."""
    of = o.float()
    nrm = (of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + eps)).to(BF16)
    y = w * nrm
    return (y * F.silu(z.float())).to(BF16)


class GdnLayer:
    """One layer's device state as the kernel keeps it, with the pass semantics above."""

    def __init__(self, hk: int, hv: int, conv_w: torch.Tensor, A_log: torch.Tensor,
                 dt_bias: torch.Tensor, norm_w: torch.Tensor, eps: float = 1e-6):
        assert hv % hk == 0
        self.hk, self.hv, self.eps = hk, hv, eps
        self.C = conv_dim(hk, hv)
        self.conv_w = conv_w.reshape(self.C, 4).to(BF16)
        self.A_log, self.dt_bias, self.norm_w = A_log.to(BF16), dt_bias.to(BF16), norm_w.to(BF16)
        self.ring = torch.zeros(RING, self.C, dtype=BF16)
        self.S = torch.zeros(hv, DK, DV, dtype=F32)
        self.st_k = torch.zeros(MAXN, hv, DK, dtype=F32)
        self.st_v = torch.zeros(MAXN, hv, DV, dtype=F32)
        self.st_g = torch.zeros(MAXN, hv, 2, dtype=F32)
        self.pos = 0
        self.pending = 0

    def _hist(self, P: int, t: int, qkv: torch.Tensor) -> torch.Tensor:
        cols = []
        for back in (3, 2, 1):
            tt, p = t - back, P + t - back
            if tt >= 0:
                cols.append(qkv[tt])
            elif p >= 0:
                cols.append(self.ring[p % RING])
            else:
                cols.append(torch.zeros(self.C, dtype=BF16))
        return torch.stack(cols, dim=-1)

    def step_n(self, qkv, z, b, a) -> torch.Tensor:
        """One pass over rows [n, ...] (bf16); returns the outputs [n, Hv*128] bf16."""
        n = qkv.shape[0]
        assert 1 <= n <= MAXN
        qkv, z, b, a = (t.to(BF16) for t in (qkv, z, b, a))
        P = self.pos
        for t in range(self.pending):  # 1. replay the kept rows of the previous pass
            delta_update(self.S, self.st_k[t], self.st_v[t], self.st_g[t, :, 0], self.st_g[t, :, 1])
        S = self.S.clone()  # 2. new rows advance a copy only
        out = torch.empty(n, self.hv * DV, dtype=BF16)
        for t in range(n):
            y = conv_silu(self._hist(P, t, qkv), qkv[t], self.conv_w)
            q, k, v = split_heads(y, self.hk, self.hv)
            decay, beta = gates(b[t], a[t], self.A_log, self.dt_bias)
            self.st_k[t], self.st_v[t] = k, v
            self.st_g[t, :, 0], self.st_g[t, :, 1] = decay, beta
            delta_update(S, k, v, decay, beta)
            o = read_out(S, q)
            out[t] = gated_rmsnorm(o, z[t].view(self.hv, DV), self.norm_w, self.eps).reshape(-1)
        for t in range(n):
            self.ring[(P + t) % RING] = qkv[t]
        self.pending = 0  # replayed; the caller's keep() sets the next pass's pending rows
        return out

    def keep(self, m: int) -> None:
        """The engine's bookkeeping after a pass: m rows kept (tests/test_kernels.py:194-195)."""
        self.pos += m
        self.pending = m

    def committed_state(self) -> torch.Tensor:
        """The state after every kept row (replays the pending rows on a copy)."""
        S = self.S.clone()
        for t in range(self.pending):
            delta_update(S, self.st_k[t], self.st_v[t], self.st_g[t, :, 0], self.st_g[t, :, 1])
        return S


def sequential(layer: GdnLayer, qkv, z, b, a) -> torch.Tensor:
    """Plain decode: one 1-row pass per token, each kept."""
    outs = []
    for t in range(qkv.shape[0]):
        outs.append(layer.step_n(qkv[t:t + 1], z[t:t + 1], b[t:t + 1], a[t:t + 1]))
        layer.keep(1)
    return torch.cat(outs)
