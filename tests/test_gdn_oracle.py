"""CPU pins for the Gated DeltaNet oracle (oracle/gdn_oracle.py).

Independent routes it is checked against:
  * HF transformers' qwen3_5 functions (causal_conv1d_update, torch_recurrent_gated_delta_rule,
    Qwen3_5RMSNormGated), which python/qengine/reference.py:211-242 says it mirrors, composed as
    Qwen3_5GatedDeltaNet.forward composes them for cached decode (q/k passed in fp32, as the
    reference's deltanet_core normalises them in fp32);
  * HF's chunked delta rule (a different algorithm: WY form in 64-token chunks);
  * the explicit fp64 matrix form S_t = g (I - beta k k^T) S_{t-1} + beta k v^T;
  * numpy's convolution for the causal conv; closed forms for gates and the gated norm;
  * the lazy-rollback invariant: any pattern of n-row passes with kept prefixes equals plain
    one-row decoding of the kept tokens, bit for bit (outputs and committed state).
Planted mistakes (a tiled head mapping, decay applied after the read) fail these routes."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_oracle as G

HF = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
BF = torch.bfloat16


def make_layer(hk, hv, seed=0):
    g = torch.Generator().manual_seed(seed)
    C = G.conv_dim(hk, hv)
    conv_w = (torch.randn(C, 4, generator=g) * 0.5).to(BF)
    A_log = (torch.rand(hv, generator=g) * 5.7 - 3).to(BF)
    dt_bias = torch.randn(hv, generator=g).to(BF)
    norm_w = (1 + 0.2 * torch.randn(128, generator=g)).to(BF)
    return G.GdnLayer(hk, hv, conv_w, A_log, dt_bias, norm_w)


def make_rows(L, n, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(n, L.C, generator=g) * 2).to(BF)
    z = torch.randn(n, L.hv * 128, generator=g).to(BF)
    b = (torch.randn(n, L.hv, generator=g) * 2).to(BF)
    a = (torch.randn(n, L.hv, generator=g) * 3).to(BF)
    return qkv, z, b, a


def hf_decode(L, qkv, z, b, a):
    """HF's cached single-token decode, token by token, from a fresh state."""
    hk, hv, C = L.hk, L.hv, L.C
    conv_state = torch.zeros(1, C, 3, dtype=BF)
    S = torch.zeros(1, hv, 128, 128)
    norm = HF.Qwen3_5RMSNormGated(128, eps=L.eps)
    norm.weight = torch.nn.Parameter(L.norm_w.clone())
    outs = []
    for t in range(qkv.shape[0]):
        y = HF.causal_conv1d_update(qkv[t].view(1, C, 1), conv_state, L.conv_w, None, "silu")
        y = y.view(C)
        q = y[: hk * 128].view(1, 1, hk, 128)
        k = y[hk * 128: 2 * hk * 128].view(1, 1, hk, 128)
        v = y[2 * hk * 128:].view(1, 1, hv, 128)
        beta = b[t].view(1, 1, hv).sigmoid()
        g = -L.A_log.float().exp() * F.softplus(a[t].float() + L.dt_bias)
        r = hv // hk
        q, k = q.repeat_interleave(r, dim=2), k.repeat_interleave(r, dim=2)
        o, S = HF.torch_recurrent_gated_delta_rule(q.float(), k.float(), v, g.view(1, 1, hv), beta,
                                                   initial_state=S, output_final_state=True,
                                                   use_qk_l2norm_in_kernel=True)
        o = o.to(BF).reshape(hv, 128)
        outs.append(norm(o, z[t].view(hv, 128)).reshape(-1))
    return torch.stack(outs), S[0]


def close_bf16(out, ref):
    """The reference's own tolerance for this op (tests/test_kernels.py:250-252)."""
    d = (out.float() - ref.float()).abs()
    ok = (d <= 2.0 ** -6 * ref.float().abs() + 1e-3).all()
    frac = (d > 2.0 ** -7 * ref.float().abs() + 1e-6).float().mean().item()
    return bool(ok) and frac < 0.01, d.max().item(), frac


@pytest.mark.parametrize("hk,hv", [(2, 2), (1, 3), (2, 4)])
def test_sequential_equals_hf_decode(hk, hv):
    L = make_layer(hk, hv, seed=hk * 10 + hv)
    rows = make_rows(L, 20, seed=1)
    out = G.sequential(L, *rows)
    ref, S_ref = hf_decode(L, *rows)
    ok, mx, frac = close_bf16(out, ref)
    assert ok, (mx, frac)
    assert frac < 0.002  # same rounding points: nearly every element is the same bf16
    torch.testing.assert_close(L.committed_state(), S_ref, rtol=1e-5, atol=1e-6)


def test_tiled_head_mapping_is_detected():
    """A plausible slip (q/k head j % Hk instead of j // r) is far outside the tolerance."""
    L = make_layer(2, 4, seed=5)
    rows = make_rows(L, 6, seed=2)
    ref, _ = hf_decode(L, *rows)
    orig = G.split_heads

    def tiled(y, hk, hv):
        r = hv // hk
        q = y[: hk * 128].view(hk, 128).repeat(r, 1)
        k = y[hk * 128: 2 * hk * 128].view(hk, 128).repeat(r, 1)
        v = y[2 * hk * 128:].view(hv, 128)
        return G.l2norm(q.float()) / math.sqrt(128), G.l2norm(k.float()), v.float()

    G.split_heads = tiled
    try:
        bad = G.sequential(make_layer(2, 4, seed=5), *rows)
    finally:
        G.split_heads = orig
    assert not close_bf16(bad, ref)[0]


def _delta_seq(q, k, v, decay, beta, S0):
    S, outs = S0.clone(), []
    for t in range(q.shape[0]):
        G.delta_update(S, k[t], v[t], decay[t], beta[t])
        outs.append((S * q[t][:, :, None]).sum(dim=1))
    return torch.stack(outs), S


def _qkvgb(T, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = G.l2norm(torch.randn(T, H, 128, generator=g)) / math.sqrt(128)
    k = G.l2norm(torch.randn(T, H, 128, generator=g))
    v = torch.randn(T, H, 128, generator=g)
    decay = torch.exp(-torch.rand(T, H, generator=g) * 0.5)
    beta = torch.rand(T, H, generator=g)
    return q, k, v, decay, beta


def test_delta_rule_equals_hf_chunked_form():
    """70 tokens (one full 64-chunk and a partial one) against HF's chunked algorithm."""
    T, H = 70, 3
    q, k, v, decay, beta = _qkvgb(T, H, seed=3)
    S0 = torch.randn(H, 128, 128, generator=torch.Generator().manual_seed(4)) * 0.1
    o, S = _delta_seq(q, k, v, decay, beta, S0)
    # HF scales q by 1/sqrt(dk) itself: hand it the unscaled q
    o_hf, S_hf = HF.torch_chunk_gated_delta_rule(
        (q * math.sqrt(128))[None], k[None], v[None], torch.log(decay)[None], beta[None],
        initial_state=S0[None], output_final_state=True, use_qk_l2norm_in_kernel=False)
    torch.testing.assert_close(o, o_hf[0].float(), rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(S, S_hf[0], rtol=2e-4, atol=2e-5)


def test_delta_rule_equals_fp64_matrix_form():
    T, H = 9, 2
    q, k, v, decay, beta = _qkvgb(T, H, seed=5)
    S0 = torch.randn(H, 128, 128, generator=torch.Generator().manual_seed(6)) * 0.1
    o, S = _delta_seq(q, k, v, decay, beta, S0)
    Sd = S0.double()
    I = torch.eye(128, dtype=torch.float64)
    for t in range(T):
        for h in range(H):
            kk = k[t, h].double()[:, None]
            A = decay[t, h].double() * (I - beta[t, h].double() * kk @ kk.T)
            Sd[h] = A @ Sd[h] + beta[t, h].double() * kk @ v[t, h].double()[None]
        ot = torch.einsum("hkd,hk->hd", Sd, q[t].double())
        torch.testing.assert_close(o[t].double(), ot, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(S.double(), Sd, rtol=1e-4, atol=1e-5)


def test_decay_after_the_read_is_detected():
    """Decaying S after kv = S^T k (a plausible reordering) breaks the fp64 matrix form."""
    T, H = 4, 1
    q, k, v, decay, beta = _qkvgb(T, H, seed=7)
    S = torch.randn(H, 128, 128, generator=torch.Generator().manual_seed(8))
    ref = S.clone()
    for t in range(T):
        G.delta_update(ref, k[t], v[t], decay[t], beta[t])
        kv = (S * k[t][:, :, None]).sum(dim=1)
        S.mul_(decay[t][:, None, None])
        S.add_(k[t][:, :, None] * ((v[t] - kv) * beta[t][:, None])[:, None, :])
    assert (S - ref).abs().max() > 1e-2


def test_delta_rule_closed_forms():
    H = 2
    g = torch.Generator().manual_seed(9)
    S = torch.randn(H, 128, 128, generator=g)
    k = G.l2norm(torch.randn(H, 128, generator=g))
    v = torch.randn(H, 128, generator=g)
    # beta = 1, decay = 1: the state now maps k to v exactly (up to fp32 rounding)
    S1 = S.clone()
    G.delta_update(S1, k, v, torch.ones(H), torch.ones(H))
    torch.testing.assert_close((S1 * k[:, :, None]).sum(1), v, rtol=1e-4, atol=1e-4)
    # beta = 0: pure decay
    S2 = S.clone()
    G.delta_update(S2, k, v, torch.full((H,), 0.75), torch.zeros(H))
    assert torch.equal(S2, S * 0.75)


def test_gates_closed_forms():
    hv = 4
    b = torch.tensor([0.0, 100.0, -100.0, 1.0]).to(BF)
    a = torch.tensor([30.0, 0.0, -40.0, 2.0]).to(BF)
    A_log = torch.tensor([0.0, 1.0, -2.0, 0.5]).to(BF)
    dt = torch.tensor([0.0, 0.5, 1.0, -1.0]).to(BF)
    decay, beta = G.gates(b, a, A_log, dt)
    assert beta.tolist()[:3] == [0.5, 1.0, 0.0]
    # softplus threshold: x = 30 > 20 passes through, decay = exp(-exp(0) * 30)
    assert decay[0].item() == pytest.approx(math.exp(-30.0), rel=1e-6)
    x = 0.0 + 0.5
    assert decay[1].item() == pytest.approx(math.exp(-math.e * math.log1p(math.exp(x))), rel=1e-6)
    assert decay[2].item() == pytest.approx(1.0, abs=1e-6)  # softplus(-39) ~ 1e-17
    assert hv == len(decay)


def test_conv_equals_numpy_convolution():
    """The ring-fed causal conv over a sequence equals np.convolve per channel (pre-rounding)."""
    L = make_layer(1, 1, seed=11)
    T = 23  # wraps the 16-slot ring
    qkv, z, b, a = make_rows(L, T, seed=12)
    got = []
    for t in range(T):
        hist = L._hist(L.pos, 0, qkv[t:t + 1])
        acc = (torch.cat([hist, qkv[t][:, None]], -1).double() * L.conv_w.double()).sum(-1)
        got.append(acc)
        L.step_n(qkv[t:t + 1], z[t:t + 1], b[t:t + 1], a[t:t + 1])
        L.keep(1)
    got = torch.stack(got).numpy()
    x = qkv.double().numpy()
    w = L.conv_w.double().numpy()
    for c in range(0, L.C, 37):
        want = np.convolve(x[:, c], w[c, ::-1])[:T]
        assert np.allclose(got[:, c], want, rtol=1e-12, atol=1e-12), c


def test_gated_rmsnorm_closed_form():
    o = torch.full((2, 128), 3.0).to(BF)
    o[1] = -0.5
    z = torch.full((2, 128), 20.0).to(BF)  # silu(20) = 20 * sigmoid(20)
    w = torch.ones(128).to(BF)
    y = G.gated_rmsnorm(o, z, w, 1e-6).float()
    s = 20.0 / (1 + math.exp(-20.0))
    assert torch.allclose(y[0], torch.full((128,), s).to(BF).float())
    assert torch.allclose(y[1], torch.full((128,), -s).to(BF).float())


@pytest.mark.parametrize("hk,hv", [(2, 2), (1, 3)])
def test_passes_with_rollback_equal_plain_decode(hk, hv):
    """n-row passes keeping a prefix reproduce one-row decoding of the kept tokens exactly."""
    spec, plain = make_layer(hk, hv, seed=13), make_layer(hk, hv, seed=13)
    rng = torch.Generator().manual_seed(14)
    for it, n in enumerate([8, 1, 3, 8, 2, 5, 1, 7, 4, 8, 6]):
        rows = make_rows(spec, n, seed=100 + it)
        keep = int(torch.randint(1, n + 1, (1,), generator=rng))
        out = spec.step_n(*rows)
        spec.keep(keep)
        for t in range(keep):
            o1 = plain.step_n(*(r[t:t + 1] for r in rows))
            plain.keep(1)
            assert torch.equal(out[t], o1[0]), (it, t)
    assert spec.pos == plain.pos > 16  # the ring wrapped
    assert torch.equal(spec.committed_state(), plain.committed_state())


def test_rejected_rows_leave_no_trace():
    """A pass whose rows are all rejected but the first leaves the same future as never having
    seen the rejected rows (stale ring slots are rewritten before they are read)."""
    A, B = make_layer(2, 2, seed=15), make_layer(2, 2, seed=15)
    r1 = make_rows(A, 6, seed=16)
    A.step_n(*r1)
    A.keep(1)
    B.step_n(*(r[:1] for r in r1))
    B.keep(1)
    for it in range(4):
        rows = make_rows(A, 3, seed=200 + it)
        assert torch.equal(A.step_n(*rows), B.step_n(*rows))
        A.keep(3)
        B.keep(3)


def test_nan_stays_in_its_head():
    L = make_layer(2, 2, seed=17)
    qkv, z, b, a = make_rows(L, 1, seed=18)
    qkv[0, 2 * 256 + 128 + 5] = float("nan")  # a v channel of value head 1
    out = L.step_n(qkv, z, b, a)
    assert torch.isnan(out[0, 128:]).all()
    assert not torch.isnan(out[0, :128]).any()
