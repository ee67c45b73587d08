"""GPU tests of the fused attn_prep_decode op (prep + decode in two launches): q_out, the written
KV cache rows and the attention output must be bit-identical to attn_prep followed by
attn_decode on the same inputs, and so inherit those ops' parity with the oracle (checked here
too, at the decode bar: |out-ref| <= 2^-6|ref| + 2e-3, reference tests/test_kernels.py:353)."""
import pytest
import torch

import oracle as O
from attn_cases import BF, D, attn_close, gen, norm_weights, proj_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(hq, hkv, n, pos, max_len, seed, rd=64):
    g = gen(seed)
    kc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    vc = torch.randn(hkv, max_len, D, generator=g).to(BF)
    pr = proj_rows(g, n, hq, hkv)
    qnw, knw = norm_weights(g)
    inv = O.rope_inv_freq(1e7, rd)
    return kc, vc, pr, qnw, knw, inv


def _run(C, fused, kc, vc, pr, qnw, knw, inv, pos, hq, ns):
    n = pr.proj.shape[0]
    proj = pr.proj.to(DEV)
    w = hq * 2 * D
    qg, k, v = proj[:, :w], proj[:, w: w + pr.hkv * D], proj[:, w + pr.hkv * D: w + 2 * pr.hkv * D]
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    q = torch.full((n, hq * D), float("nan"), dtype=BF, device=DEV)
    out = torch.full((n, hq * D), float("nan"), dtype=BF, device=DEV)
    po = torch.empty(n, hq, ns, D, device=DEV)
    pml = torch.empty(n, hq, ns, 2, device=DEV)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    args = (qg, k, v, qnw.to(DEV), knw.to(DEV), inv.to(DEV), p, q, kcd, vcd, 1e-6)
    if fused:
        C.attn_prep_decode(*args, po, pml, out)
    else:
        C.attn_prep(*args)
        C.attn_decode(q, kcd, vcd, p, qg, po, pml, out)
    torch.cuda.synchronize()
    return q.cpu(), kcd.cpu(), vcd.cpu(), out.cpu()


@pytest.mark.parametrize("hq,hkv,n,pos,max_len,ns", [
    (24, 4, 1, 1023, 1024, 32),       # BASELINE cfg 1 shape: the new row is the cache's last
    (24, 4, 2, 4000, 8192, 64),       # cache longer than the attended prefix
    (24, 4, 5, 4096, 4101, 16),       # MTP verify shape (two column tiles: runs the two ops)
    (24, 4, 8, 4096, 4104, 16),       # three column tiles: runs prep + decode inside the op
    (8, 2, 3, 30, 100, 4),            # new rows straddle a slice boundary (slices of 32)
    (6, 1, 4, 62, 64, 2),             # rows past the end of the cache are not written
    (4, 4, 1, 0, 16, 1),              # first position, no GQA
    (24, 4, 2, 131070, 131072, 64),   # long cache
    (24, 4, 2, 2047, 4096, 64),       # rows straddle a slice-size change (32 | 64): two passes
    (24, 4, 5, 2046, 2100, 64),       # the same with two column tiles
    (24, 4, 1, 16383, 16384, 64),     # the new row in a wave's second tile (loaded after the prep)
    (24, 4, 2, 8190, 8192, 64),       # two new rows in a tile loaded before the prep (patched)
])
def test_prep_decode_equals_prep_then_decode(native, hq, hkv, n, pos, max_len, ns):
    kc, vc, pr, qnw, knw, inv = _inputs(hq, hkv, n, pos, max_len, seed=hq * 100 + n)
    a = _run(native, False, kc, vc, pr, qnw, knw, inv, pos, hq, ns)
    b = _run(native, True, kc, vc, pr, qnw, knw, inv, pos, hq, ns)
    for name, x, y in zip(("q_out", "kc", "vc", "out"), a, b):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16)), name
    # and the result is the oracle's prep + attention
    kr, vr = kc.clone(), vc.clone()
    w = hq * 2 * D
    qg = pr.proj[:, :w]
    q_ref = O.attn_prep(qg, pr.proj[:, w: w + hkv * D], pr.proj[:, w + hkv * D: w + 2 * hkv * D],
                        qnw, knw, inv, pos, kr, vr, 1e-6, hq)
    ref = O.attn_decode(q_ref, kr, vr, pos, qg, hq)
    ok, mx, mean = attn_close(b[3], ref)
    assert ok, (mx, mean)


@pytest.mark.parametrize("rd", [32, 128, 256])
def test_prep_decode_rotary_widths(native, rd):
    hq, hkv, n, pos, max_len, ns = 8, 2, 2, 200, 512, 8
    kc, vc, pr, qnw, knw, inv = _inputs(hq, hkv, n, pos, max_len, seed=rd + 7, rd=rd)
    a = _run(native, False, kc, vc, pr, qnw, knw, inv, pos, hq, ns)
    b = _run(native, True, kc, vc, pr, qnw, knw, inv, pos, hq, ns)
    for name, x, y in zip(("q_out", "kc", "vc", "out"), a, b):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16)), name


def test_prep_decode_graph_replays(native):
    """Captured once, replayed with the position advanced between replays (the engine's decode
    loop): every replay matches the unfused ops run eagerly on the same state."""
    C = native
    hq, hkv, max_len, ns = 24, 4, 2048, 64
    kc, vc, pr, qnw, knw, inv = _inputs(hq, hkv, 1, 0, max_len, seed=11)
    proj = pr.proj.to(DEV)
    w = hq * 2 * D
    qg, k, v = proj[:, :w], proj[:, w: w + hkv * D], proj[:, w + hkv * D: w + 2 * hkv * D]
    dq, dk, dinv = qnw.to(DEV), knw.to(DEV), inv.to(DEV)
    kc_f, vc_f = kc.to(DEV), vc.to(DEV)
    kc_u, vc_u = kc_f.clone(), vc_f.clone()
    pos = torch.tensor([1500], dtype=torch.int32, device=DEV)
    q_f = torch.empty(1, hq * D, dtype=BF, device=DEV)
    out_f = torch.empty_like(q_f)
    q_u, out_u = torch.empty_like(q_f), torch.empty_like(q_f)
    po, pml = torch.empty(1, hq, ns, D, device=DEV), torch.empty(1, hq, ns, 2, device=DEV)
    po2, pml2 = torch.empty_like(po), torch.empty_like(pml)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C.attn_prep_decode(qg, k, v, dq, dk, dinv, pos, q_f, kc_f, vc_f, 1e-6, po, pml, out_f)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        C.attn_prep_decode(qg, k, v, dq, dk, dinv, pos, q_f, kc_f, vc_f, 1e-6, po, pml, out_f)
    for p in (1500, 1501, 1502, 1700, 2047):
        pos.fill_(p)
        graph.replay()
        C.attn_prep(qg, k, v, dq, dk, dinv, pos, q_u, kc_u, vc_u, 1e-6)
        C.attn_decode(q_u, kc_u, vc_u, pos, qg, po2, pml2, out_u)
        torch.cuda.synchronize()
        assert torch.equal(q_f.view(torch.int16), q_u.view(torch.int16)), p
        assert torch.equal(out_f.view(torch.int16), out_u.view(torch.int16)), p
        assert torch.equal(kc_f.view(torch.int16), kc_u.view(torch.int16)), p
