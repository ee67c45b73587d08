"""CPU pin of the attention oracle against HF transformers' own gated attention.

The reference's oracle mirrors HF's qwen3_5 attention (python/qengine/reference.py:3-6,252-272).
Its HF-parity tests need model directories that are not here (test_27b_attention_layer3,
test_rope_matches_hf_mrope). The installed transformers 5.15 has `Qwen3_5Attention`, so a layer
is built from a local config with random weights: head_dim 256, partial rotary 0.25 (64 dims),
theta 1e7, 4 q heads over 2 KV heads, an identity o_proj. The whole causal sequence then goes
through both HF and this build's oracle (attn_prep + attn_decode, i.e. prefill as one-row decode
steps). The two differ only in where bf16 rounds: HF rounds scores and probabilities to bf16
inside its eager matmuls, while the oracle keeps fp32 like the reference. The bound is therefore
the reference's own HF bar (rel-L2 < 2e-2 and every row's cosine > 0.999,
test_27b_layers.py:161-162). A swapped q/gate split
and a tiled GQA head mapping each exceed it by far. The RoPE tables and the q/k norm are equal
bit for bit."""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle as O

HF = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
CFG = pytest.importorskip("transformers.models.qwen3_5.configuration_qwen3_5")
BF = torch.bfloat16
HQ, HKV, D, T = 4, 2, 256, 40


def build(seed=0):
    torch.manual_seed(seed)
    c = CFG.Qwen3_5TextConfig(
        hidden_size=HQ * D, num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
        rms_norm_eps=1e-6, attention_bias=False, max_position_embeddings=4096,
        rope_parameters={"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25,
                         "mrope_section": [11, 11, 10]})
    c._attn_implementation = "eager"
    att = HF.Qwen3_5Attention(c, 0)
    with torch.no_grad():
        for lin in (att.q_proj, att.k_proj, att.v_proj):
            lin.weight.normal_(0, 1 / math.sqrt(HQ * D))
        att.o_proj.weight.copy_(torch.eye(HQ * D))
        att.q_norm.weight.normal_(0, 0.3)
        att.k_norm.weight.normal_(0, 0.3)
    att = att.to(BF).eval()
    rot = HF.Qwen3_5TextRotaryEmbedding(c)
    x = torch.randn(1, T, HQ * D).to(BF)
    return att, rot, x


def hf_forward(att, rot, x):
    pos = torch.arange(T)[None]
    cos, sin = rot(x, pos)
    mask = torch.full((T, T), float("-inf")).triu(1)[None, None].to(BF)
    with torch.no_grad():
        out, _ = att(x, (cos, sin), mask)
    return out[0], cos[0], sin[0]


def projections(att, x):
    with torch.no_grad():
        return (F.linear(x[0], att.q_proj.weight), F.linear(x[0], att.k_proj.weight),
                F.linear(x[0], att.v_proj.weight))


def oracle_prep(att, qg, k, v):
    kc = torch.zeros(HKV, T, D, dtype=BF)
    vc = torch.zeros(HKV, T, D, dtype=BF)
    q = O.attn_prep(qg, k, v, att.q_norm.weight.detach(), att.k_norm.weight.detach(),
                    O.rope_inv_freq(1e7, 64), 0, kc, vc, 1e-6, HQ)
    return q, kc, vc


def oracle_forward(att, x, swap_gate=False, prefill=False):
    qg, k, v = projections(att, x)
    if swap_gate:  # a plausible slip: gate taken from the first half of each head's slice
        h = qg.reshape(T, HQ, 2, D)
        qg = torch.cat([h[:, :, 1], h[:, :, 0]], dim=-1).reshape(T, -1)
    q, kc, vc = oracle_prep(att, qg, k, v)
    if prefill:
        return O.attn_prefill(q, kc, vc, 0, qg, HQ)
    return O.attn_decode(q, kc, vc, 0, qg, HQ, grouped=False)


def rel_l2(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm()).item()


def min_cos(a, b):
    return F.cosine_similarity(a.float(), b.float(), dim=-1).min().item()


def test_rope_tables_equal_hf():
    att, rot, x = build()
    _, cos, sin = hf_forward(att, rot, x)
    inv = O.rope_inv_freq(1e7, 64)
    assert torch.equal(inv, rot.inv_freq)
    for p in (0, 1, 7, T - 1):
        c, s = O.rope_cos_sin(p, inv)
        assert torch.equal(c, cos[p]) and torch.equal(s, sin[p]), p


def test_qk_norm_equals_hf():
    att, rot, x = build(1)
    y = torch.randn(T, HQ, D).to(BF)
    with torch.no_grad():
        assert torch.equal(O.rmsnorm1p(y, att.q_norm.weight, 1e-6), att.q_norm(y))


@pytest.mark.parametrize("prefill", [False, True])
def test_gated_attention_matches_hf(prefill):
    att, rot, x = build(2)
    ref, _, _ = hf_forward(att, rot, x)
    out = oracle_forward(att, x, prefill=prefill)
    err, cos = rel_l2(out, ref), min_cos(out, ref)
    assert err < 2e-2 and cos > 0.999, (err, cos)
    # a swapped q/gate split is far outside the bar
    assert rel_l2(oracle_forward(att, x, swap_gate=True, prefill=prefill), ref) > 0.3


def test_gqa_head_mapping_is_pinned():
    """Replacing the GQA mapping h // grp by h % Hkv (the reference's own negative control)
    is detected against HF."""
    att, rot, x = build(3)
    ref, _, _ = hf_forward(att, rot, x)
    qg, k, v = projections(att, x)
    q, kc, vc = oracle_prep(att, qg, k, v)
    rows = []
    for t in range(T):
        gate = qg[t].reshape(HQ, 2 * D)[:, D:]
        heads = [O.attention_core(q[t].reshape(HQ, D)[h:h + 1], gate[h], kc[h % HKV:h % HKV + 1],
                                  vc[h % HKV:h % HKV + 1], t + 1) for h in range(HQ)]
        rows.append(torch.cat(heads))
    assert rel_l2(torch.stack(rows), ref) > 0.3
    assert rel_l2(oracle_forward(att, x), ref) < 2e-2


def test_partial_rope_is_pinned():
    """Rotating all 256 dims (no partial rotary) or using theta 1e4 is detected against HF."""
    att, rot, x = build(4)
    ref, _, _ = hf_forward(att, rot, x)
    qg, k, v = projections(att, x)
    for inv in (O.rope_inv_freq(1e7, 256), O.rope_inv_freq(1e4, 64)):
        kc = torch.zeros(HKV, T, D, dtype=BF)
        vc = torch.zeros(HKV, T, D, dtype=BF)
        q = O.attn_prep(qg, k, v, att.q_norm.weight.detach(), att.k_norm.weight.detach(), inv, 0,
                        kc, vc, 1e-6, HQ)
        assert rel_l2(O.attn_decode(q, kc, vc, 0, qg, HQ), ref) > 5e-2
