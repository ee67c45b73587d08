"""GPU parity of the chunked-prefill op (attn_prep_chunk + attn_prefill) against the oracle.

Bars as for decode: per element |out-ref| <= 2^-6|ref| + 2e-3 (reference
tests/test_kernels.py:353 of qengine) and max-abs <= 2e-2, mean-abs <= 2e-3 (BASELINE gate).
Prep over a whole chunk: v exact; q/k un-rotated dims within 1 bf16 ulp, rotated dims within 2
ulps of their pair's magnitude, >= 99.9% bit-equal (attn_cases.rope_close).
"""
import pytest
import torch

import oracle as O
from attn_cases import BF, D, attn_close, gen, norm_weights, proj_rows, rope_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_prefill(C, q, kc, vc, pos, qg):
    T, hq = q.shape[0], q.shape[1] // D
    out = torch.empty(T, hq * D, dtype=BF, device=DEV)
    C.attn_prefill(q.to(DEV), kc, vc, torch.tensor([pos], dtype=torch.int32, device=DEV),
                   qg.to(DEV), out)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("hq,hkv,T,pos,max_len", [
    (24, 4, 300, 0, 300),      # chunk from an empty cache: first rows attend 1, 2, ... positions
    (8, 2, 129, 50, 179),      # ragged last row block
    (6, 1, 1, 5, 6),           # one row
    (24, 4, 128, 1000, 1100),  # cache longer than the chunk needs
    (4, 4, 64, 0, 64),         # no GQA
    (24, 4, 200, 100, 250),    # rows past the end of the cache attend the whole cache
    (12, 2, 16, 0, 16),        # GQA 6, one 16-row block (the balanced layout's half pair)
    (24, 4, 17, 3, 30),        # GQA 6, two blocks, the second ragged
    (6, 1, 48, 700, 760),      # GQA 6, one KV head, three blocks
    (24, 4, 150, 30, 180),     # GQA 6, 10 blocks: an odd number (5) of workgroups per KV head
    (6, 1, 80, 0, 80),         # GQA 6, 5 blocks (3 workgroups, the last block's quad part-empty)
])
def test_prefill_matches_oracle(native, hq, hkv, T, pos, max_len):
    g = gen(hq * 1000 + T)
    kc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    vc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    q = torch.randn(T, hq * D, generator=g).to(BF)
    qg = torch.randn(T, hq * 2 * D, generator=g).to(BF)
    out = run_prefill(native, q, kc.to(DEV), vc.to(DEV), pos, qg)
    ok, mx, mean = attn_close(out, O.attn_prefill(q, kc, vc, pos, qg, hq))
    assert ok, (mx, mean)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (24, 4)])  # the 8-wave and the balanced layout
def test_prefill_ignores_unattended_cache(native, hq, hkv):
    T, pos, max_len = 96, 40, 400
    g = gen(77 + hq)
    kc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    vc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    q = torch.randn(T, hq * D, generator=g).to(BF)
    qg = torch.randn(T, hq * 2 * D, generator=g).to(BF)
    a = run_prefill(native, q, kc.to(DEV), vc.to(DEV), pos, qg)
    kc[:, pos + T:] = float("nan")
    vc[:, pos + T:] = float("nan")
    b = run_prefill(native, q, kc.to(DEV), vc.to(DEV), pos, qg)
    assert torch.isfinite(b.float()).all() and torch.equal(a, b)


def test_config5_chunked_prefill(native):
    """cfg 5: a 2048-row chunk appended to a 2048-position cache, 24 Q / 4 KV heads, partial
    RoPE (theta 1e7, 64 dims), sigmoid gate: attn_prep_chunk writes the chunk's K/V and q, then
    attn_prefill attends causally."""
    C = native
    hq, hkv, T, pos = 24, 4, 2048, 2048
    max_len = pos + T
    g = gen(5)
    qnw, knw = norm_weights(g)
    kc = torch.zeros(hkv, max_len, D, dtype=BF)
    vc = torch.zeros_like(kc)
    kc[:, :pos] = torch.randn(hkv, pos, D, generator=g).to(BF)
    vc[:, :pos] = torch.randn(hkv, pos, D, generator=g).to(BF)
    pr = proj_rows(g, T, hq, hkv)
    inv = O.rope_inv_freq(1e7, 64)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref = O.attn_prep(pr.qg, pr.k, pr.v, qnw, knw, inv, pos, kc_ref, vc_ref, 1e-6, hq)
    ref = O.attn_prefill(q_ref, kc_ref, vc_ref, pos, pr.qg, hq)

    kc_d, vc_d, prd = kc.to(DEV), vc.to(DEV), pr.proj.to(DEV)
    qg_d = prd[:, : hq * 2 * D]
    k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
    v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
    posd = torch.tensor([pos], dtype=torch.int32, device=DEV)
    q = torch.empty(T, hq * D, dtype=BF, device=DEV)
    C.attn_prep_chunk(qg_d, k_d, v_d, qnw.to(DEV), knw.to(DEV), inv.to(DEV), posd, q, kc_d, vc_d,
                      1e-6)
    # 2048 rows x 28 heads: see rope_close for why rotated dims are judged by pair magnitude
    ok, err, frac = rope_close(q.cpu(), q_ref)
    assert ok, ("q", err, frac)
    ok, err, frac = rope_close(kc_d.cpu()[:, pos:], kc_ref[:, pos:])
    assert ok, ("k", err, frac)
    assert torch.equal(kc_d.cpu()[:, :pos], kc_ref[:, :pos])
    assert torch.equal(vc_d.cpu(), vc_ref)
    # attention on the oracle's q and cache, so the check does not depend on q/k rounding flips
    out = torch.empty(T, hq * D, dtype=BF, device=DEV)
    C.attn_prefill(q_ref.to(DEV), kc_ref.to(DEV), vc_ref.to(DEV), posd, qg_d, out)
    torch.cuda.synchronize()
    ok, mx, mean = attn_close(out.cpu(), ref)
    assert ok, (mx, mean)


@pytest.mark.parametrize("T", [9, 40, 1001])
def test_prep_chunk_equals_eight_row_preps(native, T):
    """attn_prep_chunk takes 8 rows per workgroup with a shared rotary table; attn_prep over the
    same rows in calls of at most 8 rows takes one row per workgroup. q_out and the written cache
    rows are equal bit for bit, including a ragged last block."""
    C = native
    hq, hkv, pos = 24, 4, 300
    max_len = pos + T + 5
    g = gen(T)
    qnw, knw = (w.to(DEV) for w in norm_weights(g))
    pr = proj_rows(g, T, hq, hkv)
    prd = pr.proj.to(DEV)
    qg_d = prd[:, : hq * 2 * D]
    k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
    v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
    inv = O.rope_inv_freq(1e7, 64).to(DEV)
    kc_a = torch.zeros(hkv, max_len, D, dtype=BF, device=DEV)
    vc_a, kc_b, vc_b = kc_a.clone(), kc_a.clone(), kc_a.clone()
    q_a = torch.empty(T, hq * D, dtype=BF, device=DEV)
    q_b = torch.empty_like(q_a)
    C.attn_prep_chunk(qg_d, k_d, v_d, qnw, knw, inv, torch.tensor([pos], dtype=torch.int32,
                      device=DEV), q_a, kc_a, vc_a, 1e-6)
    for t0 in range(0, T, 8):
        t1 = min(T, t0 + 8)
        C.attn_prep(qg_d[t0:t1], k_d[t0:t1], v_d[t0:t1], qnw, knw, inv,
                    torch.tensor([pos + t0], dtype=torch.int32, device=DEV), q_b[t0:t1], kc_b,
                    vc_b, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q_a.view(torch.int16), q_b.view(torch.int16))
    assert torch.equal(kc_a.view(torch.int16), kc_b.view(torch.int16))
    assert torch.equal(vc_a.view(torch.int16), vc_b.view(torch.int16))
