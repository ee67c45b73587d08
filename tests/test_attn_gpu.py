"""GPU parity tests: the gfx950 kernels vs the CPU oracle on identical seeded inputs.

Bars:
  prep   : q and k within 1 bf16 ulp of the oracle, v copied exactly (reference
           tests/test_kernels.py:341-346).
  decode : per element |out-ref| <= 2^-6|ref| + 2e-3 (reference tests/test_kernels.py:353) and
           max-abs <= 2e-2, mean-abs <= 2e-3 (BASELINE gate), fp32 accumulation.
  rows   : row t of an n-row call is bit-identical to a 1-row call at position pos+t
           (reference tests/test_kernels.py:354-357); MTP verify argmax == sequential decodes.
"""
import copy

import pytest
import torch

import oracle as O
from attn_cases import BF, D, attn_close, decode_case, gen, norm_weights, proj_rows, ulp_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(t):
    return t.to(DEV)


def gpu_decode(C, case, ns, pos=None, rows=None):
    """Run attn_decode on the GPU for `case` (optionally a row slice / other pos)."""
    q, qg = case.q, case.qg
    if rows is not None:
        q, qg = q[rows], qg[rows]
    n = q.shape[0]
    p = case.pos if pos is None else pos
    out = torch.empty(n, case.hq * D, dtype=BF, device=DEV)
    po = torch.empty(n, case.hq, ns, D, device=DEV)
    pml = torch.empty(n, case.hq, ns, 2, device=DEV)
    kc, vc = getattr(case, "_kc_dev", None), getattr(case, "_vc_dev", None)
    if kc is None:
        kc, vc = _dev(case.kc), _dev(case.vc)
        case._kc_dev, case._vc_dev = kc, vc
    C.attn_decode(_dev(q), kc, vc, torch.tensor([p], dtype=torch.int32, device=DEV), _dev(qg),
                  po, pml, out)
    torch.cuda.synchronize()
    return out.cpu()


def oracle_decode(case):
    return O.attn_decode(case.q, case.kc, case.vc, case.pos, case.qg, case.hq)


# ------------------------------------------------------------------ reference unit-test cases
@pytest.mark.parametrize("hq,hkv,steps,start,n", [(8, 2, 20, 0, 1), (24, 4, 6, 0, 1),
                                                    (8, 2, 3, 4094, 1), (1, 1, 5, 125, 1),
                                                    (8, 2, 24, 0, 8), (24, 4, 12, 100, 3)])
def test_attention_reference_cases(native, hq, hkv, steps, start, n):
    """The reference's test_attention (tests/test_kernels.py:302-357) on the oracle: passes of n
    rows at start, start+n, ...; prep vs oracle (q/k <= 1 ulp, v exact); decode on the oracle's
    cache vs oracle attention; each row bit-identical to a 1-row pass."""
    C = native
    g = gen(1)
    max_len = start + steps
    qnw, knw = norm_weights(g)
    kc = torch.zeros(hkv, max_len, D, dtype=BF)
    vc = torch.zeros_like(kc)
    kc[:, :start] = torch.randn(hkv, start, D, generator=g).to(BF)
    vc[:, :start] = torch.randn(hkv, start, D, generator=g).to(BF)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    kc_d, vc_d = _dev(kc), _dev(vc)
    inv = O.rope_inv_freq(1e7, 64)
    NS = 16
    po = torch.empty(8, hq, NS, D, device=DEV)
    pml = torch.empty(8, hq, NS, 2, device=DEV)
    pos_t = torch.zeros(1, dtype=torch.int32, device=DEV)
    for p0 in range(start, start + steps, n):
        nn = min(n, start + steps - p0)
        pr = proj_rows(g, nn, hq, hkv)
        q_ref = O.attn_prep(pr.qg, pr.k, pr.v, qnw, knw, inv, p0, kc_ref, vc_ref, 1e-6, hq)
        refs = O.attn_decode(q_ref, kc_ref, vc_ref, p0, pr.qg, hq)
        pos_t.fill_(p0)
        prd = _dev(pr.proj)
        qg_d = prd[:, : hq * 2 * D]
        k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
        v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
        q_out = torch.empty(nn, hq * D, dtype=BF, device=DEV)
        C.attn_prep(qg_d, k_d, v_d, _dev(qnw), _dev(knw), _dev(inv), pos_t, q_out, kc_d, vc_d, 1e-6)
        ok, err = ulp_close(q_out.cpu(), q_ref, ulps=1)
        assert ok, ("q", p0, err)
        ok, err = ulp_close(kc_d[:, p0:p0 + nn].cpu(), kc_ref[:, p0:p0 + nn], ulps=1)
        assert ok, ("k", p0, err)
        assert torch.equal(vc_d[:, p0:p0 + nn].cpu(), vc_ref[:, p0:p0 + nn])
        # attention on the oracle's cache so the check is independent of q/k rounding flips
        kr, vr, qr = _dev(kc_ref), _dev(vc_ref), _dev(q_ref)
        out = torch.empty(nn, hq * D, dtype=BF, device=DEV)
        C.attn_decode(qr, kr, vr, pos_t, qg_d, po, pml, out)
        for t in range(nn):
            ok, mx, mean = attn_close(out[t].cpu(), refs[t])
            assert ok, (p0 + t, mx, mean)
            o1 = torch.empty(1, hq * D, dtype=BF, device=DEV)
            C.attn_decode(qr[t:t + 1], kr, vr, pos_t + t, qg_d[t:t + 1], po, pml, o1)
            assert torch.equal(o1[0], out[t]), ("row bit-exactness", p0 + t)


# ------------------------------------------------------------------ BASELINE configurations
def test_config1_prep_and_decode(native):
    """cfg 1: one layer, one decode step at KV 1024 (pos 1023), 24 Q / 4 KV heads, theta 1e7,
    rotary 64, scale 1/16: full prep (writes position 1023) + decode."""
    C = native
    hq, hkv, L = 24, 4, 1024
    g = gen(0)
    kc = torch.zeros(hkv, L, D, dtype=BF)
    vc = torch.zeros_like(kc)
    kc[:, :L - 1] = torch.randn(hkv, L - 1, D, generator=g).to(BF)
    vc[:, :L - 1] = torch.randn(hkv, L - 1, D, generator=g).to(BF)
    qnw, knw = norm_weights(g)
    pr = proj_rows(g, 1, hq, hkv)
    inv = O.rope_inv_freq(1e7, 64)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref = O.attn_prep(pr.qg, pr.k, pr.v, qnw, knw, inv, L - 1, kc_ref, vc_ref, 1e-6, hq)
    ref = O.attn_decode(q_ref, kc_ref, vc_ref, L - 1, pr.qg, hq)
    kc_d, vc_d, prd = _dev(kc), _dev(vc), _dev(pr.proj)
    qg_d = prd[:, : hq * 2 * D]
    k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
    v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
    pos = torch.tensor([L - 1], dtype=torch.int32, device=DEV)
    q = torch.empty(1, hq * D, dtype=BF, device=DEV)
    C.attn_prep(qg_d, k_d, v_d, _dev(qnw), _dev(knw), _dev(inv), pos, q, kc_d, vc_d, 1e-6)
    NS = 16
    po = torch.empty(1, hq, NS, D, device=DEV)
    pml = torch.empty(1, hq, NS, 2, device=DEV)
    out = torch.empty(1, hq * D, dtype=BF, device=DEV)
    C.attn_decode(q, kc_d, vc_d, pos, qg_d, po, pml, out)
    ok, mx, mean = attn_close(out.cpu(), ref)
    assert ok, (mx, mean)


def _ns(ns, max_len, kv8=False):
    """A split count, or "default": the count the engine and the bench use (default_splits)."""
    import qengine_amd as qa
    return qa.default_splits(max_len, 4, kv8=kv8) if ns == "default" else ns


_ORACLE = {}


def cached_oracle(key, case):
    """The oracle's output for a case built from a seed (several split counts share it)."""
    if key not in _ORACLE:
        _ORACLE[key] = oracle_decode(case)
    return _ORACLE[key]


@pytest.mark.parametrize("L", [1024, 4096, 16384, 32768])
@pytest.mark.parametrize("ns", [16, 64, "default"])
def test_config2_split_sweep(native, L, ns):
    """cfg 2: split-KV decode at KV 4k/16k/32k (and cfg 1's 1k), N(0,1) cache, seeded, at the
    split count the bench times (default_splits: 52 on MI355X) and at 16 and 64."""
    case = decode_case(seed=L, hq=24, hkv=4, pos=L - 1, n=1)
    out = gpu_decode(native, case, _ns(ns, L))
    ok, mx, mean = attn_close(out, cached_oracle(("cfg2", L), case))
    assert ok, (L, ns, mx, mean)


@pytest.mark.parametrize("L,n", [(4096, 2), (16384, 2), (16384, 5), (32768, 3)])
def test_default_split_rows_bit_exact(native, L, n):
    """At the default split count, row t of an n-row call (one and two MFMA column tiles) equals
    a 1-row call at position pos+t bit for bit, and the call matches the oracle."""
    ns = _ns("default", L)
    case = decode_case(seed=L + n, hq=24, hkv=4, pos=L - n, n=n, max_len=L)
    out = gpu_decode(native, case, ns)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


@pytest.mark.parametrize("ns", [512, "default"])
@pytest.mark.parametrize("adversarial", [False, True])
def test_config4_long_context(native, adversarial, ns):
    """cfg 4: KV 131072 (537 MB of K+V); the adversarial variant scales 1% of key rows by 8; at
    512 splits and at the default count (the bench's)."""
    L = 131072
    case = decode_case(seed=4, hq=24, hkv=4, pos=L - 1, n=1,
                       key_scale_frac=0.01 if adversarial else 0.0)
    out = gpu_decode(native, case, _ns(ns, L))
    ok, mx, mean = attn_close(out, cached_oracle(("cfg4", adversarial), case))
    assert ok, (adversarial, ns, mx, mean)


@pytest.mark.parametrize("ns", [16, "default"])
def test_config3_mtp_verify(native, ns):
    """cfg 3: 5 rows (1 accepted + 4 drafts) at pos 4096, causal among themselves, over 4096
    cached + 5 new rows. Rows must be bit-identical to 5 sequential 1-row decodes, so argmax over a
    seeded bf16 projection [151936 x 5120] . [5120 x 6144] of the outputs is identical; both
    also stay within tolerance of the oracle. At 16 splits and at the bench's default count."""
    C = native
    case = decode_case(seed=3, hq=24, hkv=4, pos=4096, n=5, max_len=4096 + 64)
    ns = _ns(ns, case.kc.shape[1])
    verify = gpu_decode(C, case, ns)
    seq = torch.cat([gpu_decode(C, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
                     for t in range(5)])
    assert torch.equal(verify, seq)
    ref = oracle_decode(case)
    ok, mx, mean = attn_close(verify, ref)
    assert ok, (mx, mean)
    gd = torch.Generator(device=DEV).manual_seed(33)
    w_o = (torch.randn(5120, 24 * D, generator=gd, device=DEV) * (24 * D) ** -0.5).to(BF)
    w_lm = (torch.randn(151936, 5120, generator=gd, device=DEV) * 5120 ** -0.5).to(BF)

    def tokens(o):
        h = o.to(DEV) @ w_o.t()
        return (h @ w_lm.t()).float().argmax(-1).cpu()

    assert torch.equal(tokens(verify), tokens(seq))
    agree = (tokens(verify) == tokens(ref)).float().mean().item()
    assert agree >= 0.8, agree  # vs the oracle: same argmax unless two logits nearly tie


# ------------------------------------------------------------------ semantics and edge cases
@pytest.mark.parametrize("ns", [1, 3, 16, 100, 1000])
def test_split_count_does_not_matter(native, ns):
    """Any split count gives the oracle's answer (row t in slices of split_size(L_t, NS))."""
    case = decode_case(seed=7, hq=24, hkv=4, pos=3000, n=3, max_len=5000)
    ok, mx, mean = attn_close(gpu_decode(native, case, ns), oracle_decode(case))
    assert ok, (ns, mx, mean)


@pytest.mark.parametrize("hq,hkv,n", [(24, 4, 8), (8, 2, 8), (8, 1, 8), (16, 1, 4), (4, 4, 2),
                                      (32, 8, 7), (6, 1, 1)])
def test_gqa_shapes_and_rows(native, hq, hkv, n):
    """Group sizes 1..16 and 1..8 rows (1 to 4 MFMA column tiles) vs the oracle, rows bit-exact."""
    case = decode_case(seed=hq * 10 + n, hq=hq, hkv=hkv, pos=777, n=n, max_len=1000)
    out = gpu_decode(native, case, 8)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, 8, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


@pytest.mark.parametrize("hq,hkv,n,ns", [
    (24, 4, 12, 16),    # GQA 6: row chunks of 8 + 4
    (24, 4, 21, 52),    # 8 + 8 + 5 rows, the default split count of a 4-KV-head cache
    (8, 1, 9, 8),       # GQA 8: chunks of 8 + 1
    (32, 2, 6, 16),     # GQA 16: chunks of 4 + 2
    (96, 1, 2, 16),     # GQA 96: one row and 48 + 48 q heads per launch
    (130, 2, 2, 8),     # GQA 65: 32 + 33 q heads of each KV head per launch
    (66, 1, 1, 4),
])
def test_wide_calls_run_as_several_launches(native, hq, hkv, n, ns):
    """More than 8 rows or more than 64 query columns (group size x rows), which the reference
    accepts (its rows are bounded only by part_o, any group size: csrc/bindings.cpp:176-179): the
    partials run as several launches. Results match the oracle and each row is bit-identical to
    a 1-row call."""
    case = decode_case(seed=hq * 7 + n, hq=hq, hkv=hkv, pos=600, n=n, max_len=640)
    out = gpu_decode(native, case, ns)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


def test_wide_group_equals_its_sub_groups(native):
    """A 96-head group (one KV head) runs as two launches of 48 q heads: each half of the output
    equals, bit for bit, a 48-head call on the same cache with that half's q and gate rows."""
    case = decode_case(seed=96, hq=96, hkv=1, pos=1500, n=2, max_len=1600)
    out = gpu_decode(native, case, 16)
    for h0 in (0, 48):
        sub = copy.copy(case)
        sub.q = case.q[:, h0 * D:(h0 + 48) * D].contiguous()
        sub.qg = case.qg[:, h0 * 2 * D:(h0 + 48) * 2 * D].contiguous()
        sub.hq = 48
        half = gpu_decode(native, sub, 16)
        assert torch.equal(half, out[:, h0 * D:(h0 + 48) * D]), h0


@pytest.mark.parametrize("hq,hkv,n,pos,ns", [
    (24, 4, 2, 2047, 64),   # lengths 2048 | 2049: slices of 32 | 64 (one column tile)
    (24, 4, 5, 2046, 64),   # 2 + 3 rows (two column tiles)
    (24, 4, 8, 2044, 64),   # 4 + 4 rows (three column tiles, one wave per tile)
    (32, 4, 8, 2044, 64),   # four column tiles
    (24, 4, 8, 4092, 64),   # slices of 64 | 96
    (8, 2, 4, 510, 16),     # 2 + 2 rows, 16 splits
    (8, 2, 3, 30, 1),       # one split: slices of 32 | 64
])
def test_rows_straddling_a_slice_size_change(native, hq, hkv, n, pos, ns):
    """The rows of one call fall on both sides of a change of slice size (the call runs one pass
    per size): results match the oracle and each row is bit-identical to a 1-row call."""
    case = decode_case(seed=pos + n, hq=hq, hkv=hkv, pos=pos, n=n, max_len=pos + n + 40)
    out = gpu_decode(native, case, ns)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


@pytest.mark.parametrize("hq,hkv,n,pos,ns", [
    (24, 4, 8, 3000, 8),    # slices of 384: 12 tiles, 3 rounds of the 4 position subsets
    (24, 4, 6, 5000, 4),    # slices of 1280: 40 tiles, 10 rounds (the last slice: 37 tiles)
    (24, 4, 7, 4090, 16),   # slices of 256 | 288: 2 and 3 rounds, one pass per size
    (24, 4, 8, 700, 2),     # slices of 352 | 384: 11 tiles leave 3 of 4 subsets in round 3
    (32, 8, 8, 3000, 8),    # four column tiles (two per wave)
])
def test_multi_round_slices(native, hq, hkv, n, pos, ns):
    """6-8 rows (3-4 MFMA column tiles) over slices of several rounds of tiles, where each round's
    K and V loads overlap the previous half-round's arithmetic: results match the oracle and each
    row is bit-identical to a 1-row call."""
    case = decode_case(seed=pos + ns, hq=hq, hkv=hkv, pos=pos, n=n, max_len=pos + n + 24)
    out = gpu_decode(native, case, ns)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


@pytest.mark.parametrize("n,pos,ns", [(8, 3000, 200), (5, 777, 100), (6, 5000, 64), (8, 100, 3)])
def test_combine_batches_and_rows(native, n, pos, ns):
    """The combine merges slices in batches of 64 (16 lane groups of 4 slices, a fixed tree across
    the groups, the running max rescaling between batches): several batches (ns 100, 200), one
    full batch and fewer slices than one batch (ns 3) match the oracle, and row t of the n-row
    call equals a 1-row call bit for bit."""
    case = decode_case(seed=pos * 3 + n, hq=24, hkv=4, pos=pos, n=n, max_len=pos + n + 8)
    out = gpu_decode(native, case, ns)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, ns, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


@pytest.mark.parametrize("n", [3, 5])
def test_two_tile_kernels_give_the_same_bits(native, n):
    """3-5 rows (two MFMA column tiles) take the multi-column kernel when every slice of the cache
    holds at most 4 tiles (max_len <= 128 NS) and the two-tile kernel otherwise. The same call on
    caches of 8192 and 8193 positions (NS = 64) attends the same positions through both kernels:
    the outputs are equal bit for bit, match the oracle, and each row equals a 1-row call."""
    case = decode_case(seed=40 + n, hq=24, hkv=4, pos=8000, n=n, max_len=8193)
    short = copy.copy(case)
    short.kc, short.vc = case.kc[:, :8192].contiguous(), case.vc[:, :8192].contiguous()
    out_long = gpu_decode(native, case, 64)
    out_short = gpu_decode(native, short, 64)
    assert torch.equal(out_long, out_short)
    ok, mx, mean = attn_close(out_short, oracle_decode(short))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, short, 64, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out_short[t]), t


@pytest.mark.parametrize("n,pos", [(1, 1000), (5, 3000), (8, 200)])
def test_short_prefix_in_a_long_cache(native, n, pos):
    """A cache far longer than the attended prefix: slices follow the attended length (the
    reference's ceil(L/NS), attn.cu:78-80), results match the oracle and rows stay bit-exact."""
    case = decode_case(seed=n * 7 + pos, hq=24, hkv=4, pos=pos, n=n, max_len=32768)
    out = gpu_decode(native, case, 64)
    ok, mx, mean = attn_close(out, oracle_decode(case))
    assert ok, (mx, mean)
    for t in range(n):
        o1 = gpu_decode(native, case, 64, pos=case.pos + t, rows=slice(t, t + 1))
        assert torch.equal(o1[0], out[t]), t


def test_max_len_clamp(native):
    """Rows past the end of the cache attend the whole cache (attn.cu:78)."""
    case = decode_case(seed=11, hq=24, hkv=4, pos=1000, n=6, max_len=1003)
    ok, mx, mean = attn_close(gpu_decode(native, case, 4), oracle_decode(case))
    assert ok, (mx, mean)


@pytest.mark.parametrize("pos", [0, 1, 31, 32, 33, 255, 256, 257])
def test_short_prefixes(native, pos):
    """Tile and slice boundaries at short lengths, including a single attended position."""
    case = decode_case(seed=pos, hq=24, hkv=4, pos=pos, n=2, max_len=300)
    ok, mx, mean = attn_close(gpu_decode(native, case, 4), oracle_decode(case))
    assert ok, (pos, mx, mean)


def test_unattended_cache_is_never_read(native):
    """NaN in cache rows past the attended range must not reach the output."""
    clean = decode_case(seed=5, hq=24, hkv=4, pos=500, n=4, max_len=700)
    dirty = decode_case(seed=5, hq=24, hkv=4, pos=500, n=4, max_len=700)
    dirty.kc[:, 504:] = float("nan")
    dirty.vc[:, 504:] = float("nan")
    a, b = gpu_decode(native, clean, 16), gpu_decode(native, dirty, 16)
    assert torch.isfinite(b.float()).all()
    assert torch.equal(a, b)


def test_partials_then_combine_equals_decode(native):
    """attn_decode == attn_decode_partials followed by attn_decode_combine, bit for bit."""
    C = native
    case = decode_case(seed=9, hq=24, hkv=4, pos=9000, n=2, max_len=9100)
    ns = 40
    ref = gpu_decode(C, case, ns)
    q, qg, kc, vc = _dev(case.q), _dev(case.qg), _dev(case.kc), _dev(case.vc)
    pos = torch.tensor([case.pos], dtype=torch.int32, device=DEV)
    po = torch.empty(2, 24, ns, D, device=DEV)
    pml = torch.empty(2, 24, ns, 2, device=DEV)
    out = torch.empty(2, 24 * D, dtype=BF, device=DEV)
    C.attn_decode_partials(q, kc, vc, pos, qg, po, pml, out)
    C.attn_decode_combine(q, kc, vc, pos, qg, po, pml, out)
    assert torch.equal(out.cpu(), ref)


# ------------------------------------------------------------------ C ABI and graph capture
def test_capi_matches_extension(native, capi):
    """The C ABI (ctypes, no torch extension) gives the extension's bits for prep and decode."""
    C = native
    hq, hkv, max_len, n = 24, 4, 2048, 3
    g = gen(21)
    qnw, knw = norm_weights(g)
    pr = proj_rows(g, n, hq, hkv)
    inv = _dev(O.rope_inv_freq(1e7, 64))
    base = decode_case(seed=21, hq=hq, hkv=hkv, pos=1500, n=n, max_len=max_len)
    outs = []
    for path in ("ext", "capi"):
        kc, vc = _dev(base.kc), _dev(base.vc)
        prd = _dev(pr.proj)
        ldp = prd.stride(0)
        qg_d = prd[:, : hq * 2 * D]
        k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
        v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
        pos = torch.tensor([base.pos], dtype=torch.int32, device=DEV)
        q = torch.empty(n, hq * D, dtype=BF, device=DEV)
        ns = 8
        po = torch.empty(n, hq, ns, D, device=DEV)
        pml = torch.empty(n, hq, ns, 2, device=DEV)
        out = torch.empty(n, hq * D, dtype=BF, device=DEV)
        qn, kn = _dev(qnw), _dev(knw)
        if path == "ext":
            C.attn_prep(qg_d, k_d, v_d, qn, kn, inv, pos, q, kc, vc, 1e-6)
            C.attn_decode(q, kc, vc, pos, qg_d, po, pml, out)
        else:
            assert capi.prep(qg_d, k_d, v_d, ldp, qn, kn, inv, pos, q, kc, vc, n, hq, hkv,
                             max_len, 64, 1e-6) == 0
            assert capi.decode(q, kc, vc, pos, qg_d, ldp, po, pml, out, hq * D, n, hq, hkv,
                               max_len, ns) == 0
        torch.cuda.synchronize()
        outs.append((q.cpu(), kc.cpu(), vc.cpu(), out.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_graph_capture_replays(native):
    """prep + decode captured in one hipGraph, replayed at advancing positions with eager work
    in between; every replay equals the eager result (pos is read on the device)."""
    C = native
    hq, hkv, max_len, n = 24, 4, 4096, 1
    g = gen(31)
    qnw, knw = _dev(norm_weights(g)[0]), _dev(norm_weights(g)[1])
    inv = _dev(O.rope_inv_freq(1e7, 64))
    base = decode_case(seed=31, hq=hq, hkv=hkv, pos=2000, n=n, max_len=max_len)
    pr = proj_rows(g, n, hq, hkv)
    prd = _dev(pr.proj)
    qg_d = prd[:, : hq * 2 * D]
    k_d = prd[:, hq * 2 * D: hq * 2 * D + hkv * D]
    v_d = prd[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D]
    ns = 16
    po = torch.empty(n, hq, ns, D, device=DEV)
    pml = torch.empty(n, hq, ns, 2, device=DEV)

    def make_state():
        return (_dev(base.kc), _dev(base.vc), torch.empty(n, hq * D, dtype=BF, device=DEV),
                torch.empty(n, hq * D, dtype=BF, device=DEV),
                torch.tensor([base.pos], dtype=torch.int32, device=DEV))

    def step(st):
        kc, vc, q, out, pos = st
        C.attn_prep(qg_d, k_d, v_d, qnw, knw, inv, pos, q, kc, vc, 1e-6)
        C.attn_decode(q, kc, vc, pos, qg_d, po, pml, out)

    eager, graphed = make_state(), make_state()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(graphed)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    graphed[4].fill_(base.pos)
    graphed[0].copy_(_dev(base.kc))
    graphed[1].copy_(_dev(base.vc))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(graphed)
    for r in range(4):
        step(eager)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager[:4], graphed[:4]):
            assert torch.equal(a, b), r
        eager[4].add_(1)
        graphed[4].add_(1)
        torch.cuda.synchronize()


# ------------------------------------------------------------------ the engine's attention branch
def test_layer_multi_row_passes_match_token_by_token(native):
    """The reference's 27B layer test shape (tests/test_27b_layers.py:113-162 of qengine) without
    weights: passes of [1, 4, 8, 2, 8, 1, 8] rows through GatedAttention (prep + decode, the
    engine's attention branch) against the oracle run one token at a time (attention_step:
    write the cache at pos, attend [0, pos]); the caches must agree too."""
    from qengine_amd.layer import GatedAttention
    hq, hkv, T = 24, 4, 32
    g = gen(41)
    qnw, knw = norm_weights(g)
    layer = GatedAttention(hq, hkv, max_len=T, q_norm=qnw, k_norm=knw, splits=4)
    pr_all = proj_rows(g, T, hq, hkv)
    inv = O.rope_inv_freq(1e7, 64)
    kc_ref = torch.zeros(hkv, T, D, dtype=BF)
    vc_ref = torch.zeros_like(kc_ref)
    refs = []
    for t in range(T):
        q_r = O.attn_prep(pr_all.qg[t], pr_all.k[t], pr_all.v[t], qnw, knw, inv, t, kc_ref, vc_ref,
                          1e-6, hq)
        refs.append(O.attn_decode(q_r, kc_ref, vc_ref, t, pr_all.qg[t], hq)[0])
    proj_d = _dev(pr_all.proj)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    outs, t = [], 0
    for n in [1, 4, 8, 2, 8, 1, 8]:
        n = min(n, T - t)
        if n == 0:
            break
        pos.fill_(t)
        out = torch.empty(n, hq * D, dtype=BF, device=DEV)
        layer(proj_d[t:t + n], pos, out)
        outs.append(out.cpu())
        t += n
    got = torch.cat(outs)
    ok, mx, mean = attn_close(got, torch.stack(refs))
    assert ok, (mx, mean)
    ok, err = ulp_close(layer.kc.cpu(), kc_ref, ulps=1)
    assert ok, err
    assert torch.equal(layer.vc.cpu(), vc_ref)


def test_measurement_probes_run(capi):
    """The ceiling probes of the bench (measurement only: the stream probe on the partials grid
    and the grid / depth sweep) launch and return hipSuccess; the stream probes' sink stays
    untouched (the folded value never hits the sentinel on N(0,1)
    data), and an empty launch returns hipSuccess too."""
    L, hkv = 4096, 4
    g = torch.Generator(device=DEV).manual_seed(3)
    kc = torch.randn(hkv, L, D, device=DEV, generator=g).to(BF)
    vc = torch.randn(hkv, L, D, device=DEV, generator=g).to(BF)
    sink = torch.zeros(1, dtype=torch.int32, device=DEV)
    for p in (0, 100, L - 1, L + 50):
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        assert capi.kv_stream_probe(kc, vc, pos, hkv, L, 64, sink) == 0
        for gph, depth in ((1, 4), (64, 8), (512, 16), (4096, 4)):
            assert capi.kv_stream_sweep(kc, vc, pos, hkv, L, gph, depth, sink) == 0
    assert capi.launch_probe() == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
