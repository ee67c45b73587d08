"""CPU restatement of qengine's BF16 GEMV (the projections on either side of the attention path:
in_proj before attn_prep, o_proj after attn_decode). TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import this module, as the checker,
never as the measured or shipped path.

  gemv_exact(W, x)      y = x W^T in fp64: the reference test's y_exact (tests/test_kernels.py:83)
  gemv_bound(W, x)      the reference test's per-element error bound for a bf16 GEMV with fp32
                        accumulation: 2^-8 |y| + K 2^-23 sum_k |w x| (tests/test_kernels.py:84)
  gemv_bf16_ref(W, x)   the reference kernel's own arithmetic: per lane l of a 32-lane warp, fp32
                        FMAs over the 8-element chunks l, l+32, l+64, ... in that order
                        (csrc/basic.cu:113-145), then the xor-butterfly warp_sum
                        (csrc/common.cuh:58-62), lane 0's value rounded to bf16 (RNE,
                        csrc/basic.cu:147-150). bf16 x bf16 products are exact in fp32, so an fp32
                        add of the product is the FMA.

Parity pins are in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np
import torch

BF16 = torch.bfloat16


def _rows(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(1, -1) if x.dim() == 1 else x


def gemv_exact(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """[n, N] fp64: out[r][j] = sum_k W[j][k] x[r][k] (x may be one row [K])."""
    return _rows(x).double() @ W.double().t()


def gemv_bound(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """[n, N] fp64 per-element bound |y - y_exact| <= bound (tests/test_kernels.py:84)."""
    xr = _rows(x)
    K = W.shape[1]
    exact = gemv_exact(W, xr)
    return 2.0 ** -8 * exact.abs() + K * 2.0 ** -23 * (xr.double().abs() @ W.double().abs().t()) + 1e-30


def gemv_bf16_ref(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """[n, N] bf16 with the reference kernel's summation order (see the module docstring)."""
    xr = _rows(x)
    N, K = W.shape
    assert K % 8 == 0
    K8 = K // 8
    w = W.float().numpy().reshape(N, K8, 8)
    xs = xr.float().numpy().reshape(xr.shape[0], K8, 8)
    n = xs.shape[0]
    acc = np.zeros((n, N, 32), dtype=np.float32)
    for j in range((K8 + 31) // 32):           # chunk round: lane l takes chunk 32j + l
        lanes = np.arange(32)
        c = 32 * j + lanes
        live = c < K8
        cl = np.where(live, c, 0)
        for e in range(8):                      # the 8 elements of a chunk, in order
            prod = (w[None, :, cl, e] * xs[:, None, cl, e]).astype(np.float32)
            acc = np.where(live[None, None, :], (acc + prod).astype(np.float32), acc)
    for o in (16, 8, 4, 2, 1):                  # v += shfl_xor(v, o)
        acc = (acc + acc[:, :, np.arange(32) ^ o]).astype(np.float32)
    return torch.from_numpy(acc[:, :, 0].copy()).to(BF16)
