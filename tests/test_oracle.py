"""Pins for the CPU oracle (oracle/attn_oracle.py) by checks it does not share code with.

Each check is chosen so that a plausible mistake in the oracle fails it: a dropped bf16 rounding
(bit-level model), a swapped rotate-half sign or pairing (cos = 0 / sin = 1 and pos = 0 cases),
a wrong GQA head mapping or scale (brute-force fp64 loops), a wrong frequency exponent (closed
form), a wrong causal length (cache edits past the attended range), a broken split merge (any
partition of the positions gives the unsplit softmax). The reference ships no golden vectors;
tests/golden/ holds known-answer vectors computed by the same independent models.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from refmath import (attention_fp64, bf16_bits, gated_output_model, rne_bf16, rope_model,
                     sigmoid64)

BF = torch.bfloat16
D = 256


def bits(t: torch.Tensor) -> np.ndarray:
    return bf16_bits(t.float().numpy())


# ------------------------------------------------------------------------------- bf16 model
def test_rne_model_matches_torch_casts():
    """The numpy RNE model agrees with torch's float32 -> bf16 cast on random, tie and edge
    values, so it can judge the oracle's rounding points."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(100000, generator=g) * torch.exp2(torch.randint(-30, 30, (100000,), generator=g).float())
    ties = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.0 * 2 ** -8 + 1.0,
                         65504.0, 3.4e38, 1e-40, -0.0, 0.0])
    x = torch.cat([x, ties])
    want = x.to(BF).float().numpy()
    got = rne_bf16(x.numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------- RoPE
def test_inv_freq_closed_form():
    for theta, rd in ((1e7, 64), (1e4, 128), (1e6, 256), (5e5, 2)):
        inv = O.rope_inv_freq(theta, rd).double().numpy()
        want = np.array([theta ** (-2.0 * i / rd) for i in range(rd // 2)])
        assert inv[0] == 1.0
        assert np.allclose(inv, want, rtol=4e-7, atol=0), (theta, rd)


@pytest.mark.parametrize("pos", [0, 1, 7, 1023, 4096, 131071])
def test_cos_sin_tables(pos):
    inv = O.rope_inv_freq(1e7, 64)
    cos, sin = O.rope_cos_sin(pos, inv)
    assert cos.dtype == BF and cos.shape == (64,)
    assert torch.equal(cos[:32], cos[32:]) and torch.equal(sin[:32], sin[32:])
    if pos == 0:
        assert bool((cos == 1).all()) and bool((sin == 0).all())
    # fp32 angle (the reference multiplies in fp32), evaluated in fp64, rounded once to bf16
    ang = (np.float32(pos) * inv.numpy().astype(np.float32)).astype(np.float64)
    c_model = rne_bf16(np.cos(ang).astype(np.float32))
    s_model = rne_bf16(np.sin(ang).astype(np.float32))
    c_or, s_or = cos[:32].float().numpy(), sin[:32].float().numpy()
    # exact except where fp32 cos/sin (~1 ulp) straddles a bf16 rounding boundary
    for a, b in ((c_or, c_model), (s_or, s_model)):
        assert np.all(np.abs(a - b) <= 2.0 ** -8 * np.maximum(np.abs(b), 2 ** -30))
        assert np.mean(a == b) >= 0.9


def test_rope_rounding_chain_bit_exact():
    """apply_rope == the bit-level model: bf16(bf16(x*c) + bf16(rot*s)) on every element."""
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(64, 24, D, generator=g) * 3).to(BF)
    inv = O.rope_inv_freq(1e7, 64)
    for pos in (1, 17, 4095, 100000):
        cos, sin = O.rope_cos_sin(pos, inv)
        y = O.apply_rope(x, cos, sin)
        model = rope_model(x.float().numpy(), cos.float().numpy(), sin.float().numpy())
        assert np.array_equal(bits(y), bf16_bits(model)), pos


def test_rope_model_is_sensitive_to_a_dropped_rounding():
    """Negative control: skipping the intermediate roundings changes some elements, so the bit
    comparison above would catch an oracle that skipped them."""
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(4096, D, generator=g) * 3).to(BF)
    cos, sin = O.rope_cos_sin(12345, O.rope_inv_freq(1e7, 64))
    y = O.apply_rope(x, cos, sin).float().numpy()
    xf = x.float().numpy().astype(np.float64)
    c, s = cos.float().numpy().astype(np.float64), sin.float().numpy().astype(np.float64)
    once = xf.copy()
    once[:, :32] = xf[:, :32] * c[:32] - xf[:, 32:64] * s[:32]
    once[:, 32:64] = xf[:, 32:64] * c[32:] + xf[:, :32] * s[32:]
    once = rne_bf16(once.astype(np.float32))
    assert not np.array_equal(bf16_bits(once), bf16_bits(y))


def test_rope_pairing_sign_and_passthrough():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 3, D, generator=g).to(BF)
    zeros, ones = torch.zeros(64, dtype=BF), torch.ones(64, dtype=BF)
    y = O.apply_rope(x, zeros, ones)  # a quarter turn: (x1, x2) -> (-x2, x1)
    assert torch.equal(y[..., :32], -x[..., 32:64])
    assert torch.equal(y[..., 32:64], x[..., :32])
    assert torch.equal(y[..., 64:], x[..., 64:])
    assert torch.equal(O.apply_rope(x, ones, zeros), x)  # identity at pos 0


# ------------------------------------------------------------------------------- RMSNorm1p
def test_rmsnorm1p_closed_form():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(300, D, generator=g) * 3).to(BF)
    w = (0.3 * torch.randn(D, generator=g)).to(BF)
    y = O.rmsnorm1p(x, w, 1e-6).float().numpy()
    xf = x.float().numpy().astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + 1e-6)
    model = rne_bf16((xf * inv * (1.0 + w.float().numpy().astype(np.float64))).astype(np.float32))
    spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(model), 1e-30))) - 7)
    assert np.all(np.abs(y - model) <= spacing)     # within one bf16 ulp
    assert np.mean(y == model) >= 0.99              # fp32 vs fp64 rarely flips a rounding


def test_rmsnorm1p_power_of_two_scale_invariance():
    """With eps = 0, scaling x by 2^k is exact at every step, so the output is bit-identical."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, D, generator=g).to(BF)
    w = (0.3 * torch.randn(D, generator=g)).to(BF)
    base = O.rmsnorm1p(x, w, 0.0)
    for k in (-20, -3, 5, 40):
        assert torch.equal(O.rmsnorm1p((x.float() * 2.0 ** k).to(BF), w, 0.0), base)


def test_rmsnorm1p_unit_rms_with_zero_weight():
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(100, D, generator=g) * 7).to(BF)
    y = O.rmsnorm1p(x, torch.zeros(D, dtype=BF), 1e-6).float()
    rms = y.square().mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=5e-3)


# ------------------------------------------------------------------------------- q/k/v from proj
def test_qkv_from_proj_layout():
    """Each q head's slice of qg is [q | gate]; v passes through; k heads are normed + roped."""
    hq, hkv = 4, 2
    qg = torch.zeros(hq, 2 * D)
    for h in range(hq):
        qg[h, :D] = h + 1.0
        qg[h, D:] = -(h + 1.0)
    k = torch.randn(hkv * D, generator=torch.Generator().manual_seed(7)).to(BF)
    v = torch.arange(hkv * D).float().to(BF)
    inv = O.rope_inv_freq(1e7, 64)
    w0 = torch.zeros(D, dtype=BF)  # norm weight 0: scale (1 + w) = 1
    q, gate, k_out, v_out = O.attention_qkv_from_proj(qg.reshape(-1).to(BF), k, v, w0, w0, 0,
                                                      hq, hkv, 1e-6, inv)
    assert torch.equal(gate, (-torch.arange(1, hq + 1).float().repeat_interleave(D)).to(BF))
    # a constant row normalises to ~1 (exactly: x / sqrt(x^2 + eps) rounded), pos 0 = identity
    assert torch.allclose(q.float(), torch.ones(hq, D), atol=2 ** -8)
    assert torch.equal(v_out.reshape(-1), v)
    assert torch.equal(k_out, O.rmsnorm1p(k.reshape(hkv, D), w0, 1e-6))


# ------------------------------------------------------------------------------- attention
def _small_case(seed, hq, hkv, n, scale_k=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(hq, D, generator=g).to(BF)
    K = (torch.randn(hkv, n + 3, D, generator=g) * scale_k).to(BF)
    V = torch.randn(hkv, n + 3, D, generator=g).to(BF)
    gate = torch.randn(hq * D, generator=g).to(BF)
    return q, gate, K, V


@pytest.mark.parametrize("hq,hkv,n", [(4, 2, 5), (3, 1, 7), (2, 2, 1), (6, 3, 4)])
def test_attention_core_brute_force(hq, hkv, n):
    """Against explicit fp64 loops (GQA head h reads KV head h // group, scale D^-0.5)."""
    q, gate, K, V = _small_case(10 * hq + n, hq, hkv, n)
    out = O.attention_core(q, gate, K, V, n).float().numpy()
    o64 = attention_fp64(q.float().numpy(), K.float().numpy(), V.float().numpy(), hq // hkv, n,
                         D ** -0.5)
    model = gated_output_model(o64.reshape(-1), gate.float().numpy())
    spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(model), 1e-30))) - 7)
    assert np.all(np.abs(out - model) <= spacing + 1e-30)
    assert np.mean(out == model) >= 0.95


def test_attention_core_wrong_head_mapping_is_detected():
    """Negative control for the brute-force check: the tiled mapping h % hkv gives a different
    answer, so the check distinguishes the two."""
    hq, hkv, n = 4, 2, 5
    q, gate, K, V = _small_case(11, hq, hkv, n)
    out = O.attention_core(q, gate, K, V, n).float().numpy()
    Kt = K[[h % hkv for h in range(hq)]]
    Vt = V[[h % hkv for h in range(hq)]]
    o_bad = attention_fp64(q.float().numpy(), Kt.float().numpy(), Vt.float().numpy(), 1, n,
                           D ** -0.5)
    bad = gated_output_model(o_bad.reshape(-1), gate.float().numpy())
    assert np.abs(out - bad).max() > 0.05


def test_attention_uniform_and_one_hot():
    hq, hkv, n = 6, 1, 9
    g = torch.Generator().manual_seed(12)
    q = torch.randn(hq, D, generator=g).to(BF)
    V = torch.randn(hkv, n, D, generator=g).to(BF)
    gate = torch.zeros(hq * D, dtype=BF)  # sigmoid(0) = 1/2 exactly: output = bf16(o) / 2
    # all keys equal -> uniform softmax -> mean of the V rows
    K = torch.randn(hkv, 1, D, generator=g).to(BF).expand(hkv, n, D).contiguous()
    out = O.attention_core(q, gate, K, V, n).float().reshape(hq, D)
    mean_v = V.float().mean(1)
    want = rne_bf16(mean_v.numpy().astype(np.float32)) * 0.5
    assert np.allclose(out.numpy(), np.broadcast_to(want, (hq, D)), atol=2 ** -9)
    assert torch.equal(out * 2, (out * 2).to(BF).float())  # halving is exact in bf16
    # one key aligned with every query and scaled up -> softmax ~ one-hot on it
    K = torch.zeros(hkv, n, D, dtype=BF)
    K[0, 4] = (q.float().sum(0) * 8).to(BF)
    out = O.attention_core(q, gate, K, V, n).float().reshape(hq, D)
    assert torch.allclose(out, (V[0, 4].float() * 0.5).expand(hq, D), atol=2e-2)


def test_grouped_core_matches_faithful_core():
    g = torch.Generator().manual_seed(13)
    for hq, hkv, n in ((24, 4, 1000), (8, 2, 33), (4, 4, 3)):
        q = torch.randn(hq, D, generator=g).to(BF)
        K = torch.randn(hkv, n, D, generator=g).to(BF)
        V = torch.randn(hkv, n, D, generator=g).to(BF)
        gate = torch.randn(hq * D, generator=g).to(BF)
        a = O.attention_core(q, gate, K, V, n).float()
        b = O.attention_core_grouped(q, gate, K, V, n).float()
        spacing = torch.exp2(torch.floor(torch.log2(a.abs().clamp_min(1e-30))) - 7)
        assert bool(((a - b).abs() <= 2 * spacing).all())   # see test_prefill_equals_row_by_row
        assert (a == b).float().mean().item() >= 0.99


@pytest.mark.parametrize("seed", range(4))
def test_split_kv_merge_equals_unsplit(seed):
    """Flash-decoding: any partition of the positions (including empty slices) merged by
    log-sum-exp equals the unsplit softmax (exact up to fp64 rounding)."""
    rng = np.random.default_rng(seed)
    L, d = 200, 16
    q = rng.standard_normal(d)
    K = rng.standard_normal((L, d)) * (3 if seed % 2 else 1)
    V = rng.standard_normal((L, d))
    s = K @ q * 0.25
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ V
    cuts = sorted(set(rng.integers(0, L + 1, size=rng.integers(1, 12)).tolist()) | {0, L})
    bounds = list(zip(cuts[:-1], cuts[1:])) + [(L, L), (5, 5)]   # plus empty slices
    got, parts = O.flash_decode_fp64(q, K, V, 0.25, bounds)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    assert parts[-1][1] == -math.inf and parts[-1][2] == 0.0


def test_decode_rows_are_causal_and_clamped():
    """Row t attends [0, min(pos+t+1, max_len)): editing the cache past that range leaves the
    row unchanged; rows past the end of the cache attend the whole cache."""
    g = torch.Generator().manual_seed(14)
    hq, hkv, max_len, pos, n = 6, 2, 40, 30, 4
    kc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    vc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    q = torch.randn(n, hq * D, generator=g).to(BF)
    qg = torch.randn(n, hq * 2 * D, generator=g).to(BF)
    base = O.attn_decode(q, kc, vc, pos, qg, hq)
    kc2, vc2 = kc.clone(), vc.clone()
    kc2[:, pos + 1:] = 100
    vc2[:, pos + 1:] = -100
    edited = O.attn_decode(q, kc2, vc2, pos, qg, hq)
    assert torch.equal(edited[0], base[0]) and not torch.equal(edited[1], base[1])
    # clamp: pos = 38, rows 0..3 attend 39, 40, 40, 40 positions
    late = O.attn_decode(q, kc, vc, 38, qg, hq)
    assert torch.equal(late[2], O.attn_decode(q[2:3], kc, vc, 39, qg[2:3], hq)[0])
    gate = qg[3].reshape(hq, 2 * D)[:, D:].reshape(-1)
    assert torch.equal(late[3], O.attention_core_grouped(q[3].reshape(hq, D), gate, kc, vc, 40))


def test_prefill_equals_row_by_row_decode():
    g = torch.Generator().manual_seed(15)
    hq, hkv, T, pos = 8, 2, 37, 20
    kc = torch.randn(hkv, pos + T, D, generator=g).to(BF)
    vc = torch.randn(hkv, pos + T, D, generator=g).to(BF)
    q = torch.randn(T, hq * D, generator=g).to(BF)
    qg = torch.randn(T, hq * 2 * D, generator=g).to(BF)
    a = O.attn_prefill(q, kc, vc, pos, qg, hq, row_block=8).float()
    b = O.attn_decode(q, kc, vc, pos, qg, hq).float()
    # fp32 summation order differs (batched matmul vs per row): a flip of bf16(o) moves the
    # gated output by at most two bf16 ulps, and rarely
    spacing = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    assert bool(((a - b).abs() <= 2 * spacing).all())
    assert (a == b).float().mean().item() >= 0.99


def test_prep_writes_cache_below_max_len_only():
    g = torch.Generator().manual_seed(16)
    hq, hkv, max_len, n = 4, 2, 10, 3
    proj = torch.randn(n, hq * 2 * D + 2 * hkv * D, generator=g).to(BF)
    qg, k, v = proj[:, : hq * 2 * D], proj[:, hq * 2 * D: -hkv * D], proj[:, -hkv * D:]
    w = torch.zeros(D, dtype=BF)
    inv = O.rope_inv_freq(1e7, 64)
    kc = torch.full((hkv, max_len, D), 7.0, dtype=BF)
    vc = kc.clone()
    q_out = O.attn_prep(qg, k, v, w, w, inv, 8, kc, vc, 1e-6, hq)   # rows at 8, 9, 10
    assert torch.equal(vc[:, 8], v[0].reshape(hkv, D)) and torch.equal(vc[:, 9], v[1].reshape(hkv, D))
    assert bool((kc[:, :8] == 7).all())
    for t in range(n):
        q_r, _, _, _ = O.attention_qkv_from_proj(qg[t], k[t], v[t], w, w, 8 + t, hq, hkv, 1e-6, inv)
        assert torch.equal(q_out[t], q_r.reshape(-1))


def test_sigmoid_gate_rounding_points():
    """out = bf16(bf16(o) * bf16(sigmoid(g))): checked against the fp64 model on a case where
    o is exact (one attended position: o = v)."""
    g = torch.Generator().manual_seed(17)
    hq = 4
    q = torch.randn(hq, D, generator=g).to(BF)
    K = torch.randn(1, 1, D, generator=g).to(BF)
    V = torch.randn(1, 1, D, generator=g).to(BF)
    gate = (torch.randn(hq * D, generator=g) * 4).to(BF)
    out = O.attention_core(q, gate, K, V, 1).float().numpy()
    o = np.tile(V[0, 0].float().numpy(), hq).astype(np.float64)
    s = rne_bf16(sigmoid64(gate.float().numpy()).astype(np.float32)).astype(np.float64)
    model = rne_bf16((o * s).astype(np.float32))
    spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(model), 1e-30))) - 7)
    assert np.all(np.abs(out - model) <= spacing)
    assert np.mean(out == model) >= 0.99
