"""CPU pins for the GEMV oracle (oracle/gemv_oracle.py) against what the mathematics fixes:
brute-force loops, one-hot and identity closed forms, NaN propagation, the reference test's
error bound (tests/test_kernels.py:78-90 of qengine), and a literal per-lane loop of the
reference kernel (csrc/basic.cu:113-150) for the summation order."""
import numpy as np
import pytest
import torch

import oracle as O

BF = torch.bfloat16


def _rand(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(BF)


def test_exact_matches_brute_force_loops():
    g = torch.Generator().manual_seed(1)
    W, x = _rand(g, 3, 16), _rand(g, 2, 16)
    y = O.gemv_exact(W, x)
    for r in range(2):
        for j in range(3):
            want = sum(float(W[j, k]) * float(x[r, k]) for k in range(16))
            assert abs(float(y[r, j]) - want) <= 1e-12 * max(1.0, abs(want))
    assert O.gemv_exact(W, x[0]).shape == (1, 3)  # a 1-D x is one row


def _reference_loop(W: torch.Tensor, xrow: torch.Tensor, j: int) -> np.float32:
    """One output of the reference kernel, written as its loops: lane l runs chunks l, l+32, ...
    (8 elements each, fp32 FMA of exact bf16 products), then the xor butterfly; lane 0 stores."""
    K8 = W.shape[1] // 8
    v = [np.float32(0.0)] * 32
    for lane in range(32):
        acc = np.float32(0.0)
        for c in range(lane, K8, 32):
            for e in range(8):
                acc = np.float32(acc + np.float32(float(W[j, 8 * c + e]) * float(xrow[8 * c + e])))
        v[lane] = acc
    for o in (16, 8, 4, 2, 1):
        v = [np.float32(v[l] + v[l ^ o]) for l in range(32)]
    return v[0]


@pytest.mark.parametrize("N,K", [(3, 560), (2, 8), (2, 264)])
def test_reference_order_matches_its_loops(N, K):
    """The vectorised restatement of the reference's order equals the literal loops bit for bit,
    including chunk rounds where only some lanes have a chunk (K/8 not a multiple of 32)."""
    g = torch.Generator().manual_seed(K)
    W, x = _rand(g, N, K), _rand(g, 2, K)
    got = O.gemv_bf16_ref(W, x)
    for r in range(2):
        for j in range(N):
            want = torch.tensor(float(_reference_loop(W, x[r], j))).to(BF)
            assert torch.equal(got[r, j].view(torch.int16), want.view(torch.int16)), (r, j)


@pytest.mark.parametrize("N,K", [(33, 24), (127, 1000), (64, 4096), (8, 17408)])
def test_reference_order_is_within_the_bound(N, K):
    g = torch.Generator().manual_seed(N + K)
    W, x = _rand(g, N, K), _rand(g, 3, K)
    err = (O.gemv_bf16_ref(W, x).double() - O.gemv_exact(W, x)).abs()
    assert bool((err <= O.gemv_bound(W, x)).all())


def test_one_hot_and_identity_closed_forms():
    """x = e_k gives column k of W exactly; W = I gives x exactly (a single product per output is
    exact, and bf16 values survive the fp32 sum and the final rounding)."""
    g = torch.Generator().manual_seed(3)
    N, K = 40, 64
    W = _rand(g, N, K)
    for k in (0, 7, 8, 63):
        x = torch.zeros(1, K, dtype=BF)
        x[0, k] = 1.0
        assert torch.equal(O.gemv_bf16_ref(W, x)[0], W[:, k])
        assert torch.equal(O.gemv_exact(W, x)[0].to(BF), W[:, k])
    x = _rand(g, 2, K)
    eye = torch.eye(K, dtype=BF)
    assert torch.equal(O.gemv_bf16_ref(eye, x), x)


def test_transposed_weights_are_detected():
    """A plausible mistake (using W^T's layout) fails the one-hot check."""
    g = torch.Generator().manual_seed(4)
    W = _rand(g, 16, 16)
    x = torch.zeros(1, 16, dtype=BF)
    x[0, 3] = 1.0
    assert not torch.equal(O.gemv_bf16_ref(W.t().contiguous(), x)[0], W[:, 3])


def test_dropped_tail_chunk_fails_the_bound():
    """Leaving out the last 8-element chunk (a loop-bound slip) breaks the bound check."""
    g = torch.Generator().manual_seed(5)
    W, x = _rand(g, 32, 264), _rand(g, 1, 264)
    W2 = W.clone()
    W2[:, -8:] = 0
    err = (O.gemv_bf16_ref(W2, x).double() - O.gemv_exact(W, x)).abs()
    assert not bool((err <= O.gemv_bound(W, x)).all())


def test_nan_propagates_to_every_output():
    g = torch.Generator().manual_seed(6)
    W, x = _rand(g, 64, 128), _rand(g, 1, 128)
    x[0, 3] = float("nan")
    assert torch.isnan(O.gemv_bf16_ref(W, x).float()).all()
