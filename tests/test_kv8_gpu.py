"""GPU tests of the fp8 KV cache path (attn_prep_fp8, attn_decode_fp8) against the CPU oracle:
  * prep stores exactly the oracle's codes of the bf16 prep's K and V rows (value-exact), and the
    same q_out bits;
  * with scales of 1 the fp8 decode is bit-identical to the bf16 decode run on the dequantized
    cache (the MFMA inputs are the same bf16 values), which pins the fp8 tile layout and the
    conversion;
  * with any scales it is within the decode tolerance of the oracle's attention over the
    dequantized cache (per element |out-ref| <= 2^-6|ref| + 2e-3, max-abs 2e-2, mean-abs 2e-3);
  * rows of a multi-row call are bit-identical to 1-row calls, including the 6-8-row verify
    shapes that run the multi-column kernel's fp8 mode."""
import numpy as np
import pytest
import torch

import oracle as O
from attn_cases import BF, D, attn_close, decode_case
from oracle import kv8_oracle as K8

pytestmark = pytest.mark.gpu
DEV = "cuda"
F8 = torch.float8_e4m3fn


def quantize_cache(kc: torch.Tensor, scale: float) -> torch.Tensor:
    """bf16 cache -> fp8 codes (CPU oracle), as a float8_e4m3fn tensor."""
    codes = K8.encode(kc.float().numpy(), scale)
    return torch.from_numpy(codes).view(F8)


def run_fp8(C, q, qg, kc8, vc8, pos, ns, ks, vs):
    n = q.shape[0]
    hq = q.shape[1] // D
    out = torch.empty(n, hq * D, dtype=BF, device=DEV)
    po = torch.empty(n, hq, ns, D, device=DEV)
    pml = torch.empty(n, hq, ns, 2, device=DEV)
    C.attn_decode_fp8(q.to(DEV), kc8.to(DEV), vc8.to(DEV),
                      torch.tensor([pos], dtype=torch.int32, device=DEV), qg.to(DEV), po, pml,
                      out, ks, vs)
    torch.cuda.synchronize()
    return out.cpu()


def run_bf16(C, q, qg, kc, vc, pos, ns):
    n = q.shape[0]
    hq = q.shape[1] // D
    out = torch.empty(n, hq * D, dtype=BF, device=DEV)
    po = torch.empty(n, hq, ns, D, device=DEV)
    pml = torch.empty(n, hq, ns, 2, device=DEV)
    C.attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV),
                  torch.tensor([pos], dtype=torch.int32, device=DEV), qg.to(DEV), po, pml, out)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("hq,hkv,n,pos,max_len,ns", [
    (24, 4, 1, 1023, 1024, 32), (24, 4, 5, 4096, 4101, 64), (8, 2, 3, 30, 100, 4),
    (24, 4, 2, 16382, 16384, 64), (24, 4, 4, 2046, 2100, 64), (32, 8, 4, 700, 1000, 16)])
def test_fp8_scale_one_equals_bf16_on_the_dequantized_cache(native, hq, hkv, n, pos, max_len, ns):
    case = decode_case(seed=pos + n, hq=hq, hkv=hkv, pos=pos, n=n, max_len=max_len)
    kc8, vc8 = quantize_cache(case.kc, 1.0), quantize_cache(case.vc, 1.0)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)  # exact: every code is a bf16 value
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    a = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, ns, 1.0, 1.0)
    b = run_bf16(native, case.q, case.qg, kd, vd, case.pos, ns)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("hq,hkv,n,ns", [(24, 4, 13, 64), (96, 1, 2, 16), (130, 2, 1, 8)])
def test_fp8_wide_calls_equal_bf16(native, hq, hkv, n, ns):
    """More than 8 rows or more than 64 q heads per KV head over the fp8 cache (several partials
    launches): scale-1 output equals the bf16 path on the dequantized cache bit for bit."""
    case = decode_case(seed=hq + n, hq=hq, hkv=hkv, pos=900, n=n, max_len=1000)
    kc8, vc8 = quantize_cache(case.kc, 1.0), quantize_cache(case.vc, 1.0)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    a = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, ns, 1.0, 1.0)
    b = run_bf16(native, case.q, case.qg, kd, vd, case.pos, ns)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("ks,vs", [(1.0, 1.0), (0.5, 0.25), (0.037, 0.011), (3.0, 2.0)])
@pytest.mark.parametrize("n,pos,max_len", [(1, 4095, 4096), (5, 4096, 4101), (2, 300, 20000)])
def test_fp8_decode_vs_oracle(native, ks, vs, n, pos, max_len):
    case = decode_case(seed=n * 31 + pos, hq=24, hkv=4, pos=pos, n=n, max_len=max_len)
    kc8, vc8 = quantize_cache(case.kc, ks), quantize_cache(case.vc, vs)
    out = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, 64, ks, vs)
    kd = K8.dequantize(kc8.view(torch.uint8), ks)
    vd = K8.dequantize(vc8.view(torch.uint8), vs)
    ref = O.attn_decode(case.q, kd, vd, case.pos, case.qg, case.hq)
    ok, mx, mean = attn_close(out, ref)
    assert ok, (mx, mean)
    for t in range(n):
        o1 = run_fp8(native, case.q[t:t + 1], case.qg[t:t + 1], kc8, vc8, case.pos + t, 64, ks, vs)
        assert torch.equal(o1[0], out[t]), t


def test_fp8_decode_long_cache_16k(native):
    """BASELINE cfg 2's 16k shape on the fp8 cache, 1 and 5 rows, vs the oracle."""
    case = decode_case(seed=16, hq=24, hkv=4, pos=16379, n=5, max_len=16384)
    ks, vs = 0.125, 0.125
    kc8, vc8 = quantize_cache(case.kc, ks), quantize_cache(case.vc, vs)
    out = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, 64, ks, vs)
    ref = O.attn_decode(case.q, K8.dequantize(kc8.view(torch.uint8), ks),
                        K8.dequantize(vc8.view(torch.uint8), vs), case.pos, case.qg, case.hq)
    ok, mx, mean = attn_close(out, ref)
    assert ok, (mx, mean)


@pytest.mark.parametrize("ks,vs", [(1.0, 1.0), (0.05, 0.2)])
def test_prep_fp8_writes_the_oracle_codes(native, ks, vs):
    """Same q_out as attn_prep; the new K/V rows are the oracle's codes of the bf16 rows."""
    C = native
    hq, hkv, n, pos, max_len = 24, 4, 3, 500, 512
    g = torch.Generator().manual_seed(int(ks * 1000))
    proj = (torch.randn(n, hq * 2 * D + 2 * hkv * D, generator=g) * 3).to(BF).to(DEV)
    qg, k, v = proj[:, : hq * 2 * D], proj[:, hq * 2 * D: hq * 2 * D + hkv * D], proj[:, hq * 2 * D + hkv * D:]
    qnw = (torch.randn(D, generator=g) * 0.3).to(BF).to(DEV)
    knw = (torch.randn(D, generator=g) * 0.3).to(BF).to(DEV)
    inv = O.rope_inv_freq(1e7, 64).to(DEV)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    q_a, q_b = torch.empty(n, hq * D, dtype=BF, device=DEV), torch.empty(n, hq * D, dtype=BF, device=DEV)
    kc = torch.zeros(hkv, max_len, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    kc8 = torch.zeros(hkv, max_len, D, dtype=torch.uint8, device=DEV).view(F8)
    vc8 = torch.zeros_like(kc8)
    C.attn_prep(qg, k, v, qnw, knw, inv, p, q_a, kc, vc, 1e-6)
    C.attn_prep_fp8(qg, k, v, qnw, knw, inv, p, q_b, kc8, vc8, 1e-6, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(q_a, q_b)
    rows = slice(pos, pos + n)
    for cache, cache8, s in ((kc, kc8, ks), (vc, vc8, vs)):
        want = K8.decode(K8.encode(cache[:, rows].float().cpu().numpy(), s))
        got = K8.decode(cache8[:, rows].view(torch.uint8).cpu())
        assert np.array_equal(got, want)
        assert int(cache8.view(torch.uint8)[:, : pos].count_nonzero()) == 0  # nothing else written


# 6-8 rows at GQA 6 and 8 (36-64 columns) run the multi-column kernel's fp8 mode; the cases
# after the first five give slices of 3-10 rounds of tiles (partial last rounds, two passes),
# where the next round's fp8 tiles load during the current round's arithmetic
@pytest.mark.parametrize("hq,hkv,n,pos,max_len,ns", [
    (24, 4, 6, 4090, 4096, 64), (24, 4, 8, 1000, 1100, 64), (24, 4, 7, 16370, 16384, 64),
    (32, 4, 8, 600, 640, 16), (24, 4, 6, 2045, 2100, 64),
    (24, 4, 8, 3000, 3030, 8), (24, 4, 6, 5000, 5030, 4), (24, 4, 7, 4090, 4120, 16),
    (24, 4, 8, 700, 730, 2), (32, 8, 8, 3000, 3030, 8)])
def test_fp8_wide_verify_scale_one_equals_bf16(native, hq, hkv, n, pos, max_len, ns):
    case = decode_case(seed=pos + 7 * n, hq=hq, hkv=hkv, pos=pos, n=n, max_len=max_len)
    kc8, vc8 = quantize_cache(case.kc, 1.0), quantize_cache(case.vc, 1.0)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    a = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, ns, 1.0, 1.0)
    b = run_bf16(native, case.q, case.qg, kd, vd, case.pos, ns)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("ks,vs", [(0.5, 0.25), (0.037, 0.011)])
def test_fp8_wide_verify_vs_oracle_and_rows(native, ks, vs):
    """8 rows at GQA 6 against the oracle on the dequantized cache, and every row bit-identical
    to a 1-row call (which runs the one-tile kernel)."""
    n, pos, max_len = 8, 3000, 3010
    case = decode_case(seed=int(ks * 1e4), hq=24, hkv=4, pos=pos, n=n, max_len=max_len)
    kc8, vc8 = quantize_cache(case.kc, ks), quantize_cache(case.vc, vs)
    out = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, 64, ks, vs)
    ref = O.attn_decode(case.q, K8.dequantize(kc8.view(torch.uint8), ks),
                        K8.dequantize(vc8.view(torch.uint8), vs), case.pos, case.qg, case.hq)
    ok, mx, mean = attn_close(out, ref)
    assert ok, (mx, mean)
    for t in range(n):
        o1 = run_fp8(native, case.q[t:t + 1], case.qg[t:t + 1], kc8, vc8, case.pos + t, 64, ks, vs)
        assert torch.equal(o1[0], out[t]), t


def run_prefill(C, q, qg, kc, vc, pos, fp8=False, ks=1.0, vs=1.0):
    T, hq = q.shape[0], q.shape[1] // D
    out = torch.empty(T, hq * D, dtype=BF, device=DEV)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    if fp8:
        C.attn_prefill_fp8(q.to(DEV), kc.to(DEV), vc.to(DEV), p, qg.to(DEV), out, ks, vs)
    else:
        C.attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), p, qg.to(DEV), out)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("hq,hkv,T,pos", [(24, 4, 200, 300), (8, 2, 129, 0), (24, 4, 64, 2000),
                                          (16, 1, 300, 700), (8, 8, 1, 0), (6, 6, 17, 31),
                                          (24, 4, 1, 0)])
def test_prefill_fp8_scale_one_equals_bf16(native, hq, hkv, T, pos):
    """Chunked prefill over the fp8 cache with scales of 1 equals attn_prefill over the
    dequantized bf16 cache bit for bit (short rows included: they take the hi + lo P split; one
    row at position 0 is one tile, so the tile converted ahead lies past the cache)."""
    case = decode_case(seed=T + pos, hq=hq, hkv=hkv, pos=pos, n=T, max_len=pos + T + 9)
    kc8, vc8 = quantize_cache(case.kc, 1.0), quantize_cache(case.vc, 1.0)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    a = run_prefill(native, case.q, case.qg, kc8, vc8, pos, fp8=True)
    b = run_prefill(native, case.q, case.qg, kd, vd, pos)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("ks,vs", [(0.5, 0.25), (0.037, 0.011), (3.0, 2.0)])
def test_prefill_fp8_vs_oracle(native, ks, vs):
    case = decode_case(seed=int(ks * 1000), hq=24, hkv=4, pos=1000, n=300, max_len=1400)
    kc8, vc8 = quantize_cache(case.kc, ks), quantize_cache(case.vc, vs)
    out = run_prefill(native, case.q, case.qg, kc8, vc8, case.pos, fp8=True, ks=ks, vs=vs)
    kd = K8.dequantize(kc8.view(torch.uint8), ks)
    vd = K8.dequantize(vc8.view(torch.uint8), vs)
    ref = O.attn_prefill(case.q, kd, vd, case.pos, case.qg, case.hq)
    ok, mx, mean = attn_close(out, ref)
    assert ok, (mx, mean)


def test_prep_fp8_chunk_equals_eight_row_preps(native):
    """attn_prep_fp8 over 40 rows (8 rows per workgroup) writes the same q and codes as calls of
    8 rows."""
    from attn_cases import gen, norm_weights, proj_rows
    C = native
    hq, hkv, T, pos, max_len, ks, vs = 24, 4, 40, 100, 160, 0.5, 0.25
    g = gen(77)
    qnw, knw = (w.to(DEV) for w in norm_weights(g))
    prd = proj_rows(g, T, hq, hkv).proj.to(DEV)
    qg = prd[:, : hq * 2 * D]
    k = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
    v = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
    inv = O.rope_inv_freq(1e7, 64).to(DEV)
    kc_a = torch.zeros(hkv, max_len, D, dtype=torch.uint8, device=DEV).view(F8)
    vc_a, kc_b, vc_b = kc_a.clone(), kc_a.clone(), kc_a.clone()
    q_a = torch.empty(T, hq * D, dtype=BF, device=DEV)
    q_b = torch.empty_like(q_a)
    C.attn_prep_fp8(qg, k, v, qnw, knw, inv, torch.tensor([pos], dtype=torch.int32, device=DEV),
                    q_a, kc_a, vc_a, 1e-6, ks, vs)
    for t0 in range(0, T, 8):
        C.attn_prep_fp8(qg[t0:t0 + 8], k[t0:t0 + 8], v[t0:t0 + 8], qnw, knw, inv,
                        torch.tensor([pos + t0], dtype=torch.int32, device=DEV), q_b[t0:t0 + 8],
                        kc_b, vc_b, 1e-6, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(q_a.view(torch.int16), q_b.view(torch.int16))
    assert torch.equal(kc_a.view(torch.uint8), kc_b.view(torch.uint8))
    assert torch.equal(vc_a.view(torch.uint8), vc_b.view(torch.uint8))


@pytest.mark.parametrize("L", [16384, 32768])
def test_fp8_decode_default_splits(native, L):
    """The fp8 decode at the split count the bench times on an fp8 cache (default_splits with
    kv8: 64 on MI355X), one row at KV 16k / 32k: with scales of 1 bit-identical to the bf16 decode
    on the dequantized cache, and with scales of 1/8 within tolerance of the oracle."""
    import qengine_amd as qa
    ns = qa.default_splits(L, 4, kv8=True)
    case = decode_case(seed=L + 8, hq=24, hkv=4, pos=L - 1, n=1, max_len=L)
    kc8, vc8 = quantize_cache(case.kc, 1.0), quantize_cache(case.vc, 1.0)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    a = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, ns, 1.0, 1.0)
    b = run_bf16(native, case.q, case.qg, kd, vd, case.pos, ns)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ks = vs = 0.125
    kc8, vc8 = quantize_cache(case.kc, ks), quantize_cache(case.vc, vs)
    out = run_fp8(native, case.q, case.qg, kc8, vc8, case.pos, ns, ks, vs)
    ref = O.attn_decode(case.q, K8.dequantize(kc8.view(torch.uint8), ks),
                        K8.dequantize(vc8.view(torch.uint8), vs), case.pos, case.qg, case.hq)
    ok, mx, mean = attn_close(out, ref)
    assert ok, (mx, mean)


def _all_code_cache(hkv, max_len, shift):
    """fp8 cache whose values cycle through all 254 non-NaN E4M3FN codes (0x00-0x7e, 0x80-0xfe:
    zeros, subnormals, normals up to +-448), in a different order per element offset."""
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    assert codes.size == 254
    idx = (np.arange(hkv * max_len * D, dtype=np.int64) * 97 + shift) % codes.size
    return torch.from_numpy(codes[idx].reshape(hkv, max_len, D)).view(F8)


@pytest.mark.parametrize("n,pos,max_len,ns", [(1, 1200, 1201, 16), (2, 3000, 3002, 64),
                                              (5, 700, 705, 8), (7, 2000, 2007, 16)])
def test_fp8_every_code_equals_bf16(native, n, pos, max_len, ns):
    """K and V caches holding every finite E4M3FN code (the kernels' conversion runs on all of
    them: zeros, subnormals, the largest magnitudes), scales of 1: the fp8 decode (one-tile,
    two-tile and multi-column kernels) is bit-identical to the bf16 decode on the dequantized
    cache. q is scaled down so that scores against keys up to 448 stay moderate."""
    case = decode_case(seed=pos + n, hq=24, hkv=4, pos=pos, n=n, max_len=max_len)
    kc8, vc8 = _all_code_cache(4, max_len, 5), _all_code_cache(4, max_len, 71)
    kd = K8.dequantize(kc8.view(torch.uint8), 1.0).to(BF)
    vd = K8.dequantize(vc8.view(torch.uint8), 1.0).to(BF)
    q = (case.q.float() * 0.01).to(BF)
    a = run_fp8(native, q, case.qg, kc8, vc8, case.pos, ns, 1.0, 1.0)
    b = run_bf16(native, q, case.qg, kd, vd, case.pos, ns)
    assert torch.isfinite(b.float()).all()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
