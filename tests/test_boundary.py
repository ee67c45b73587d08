"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every entry point that
include/*.h declares, the C ABI rejects out-of-range arguments before launching anything,
and the torch extension enforces the reference's validation contract
(reference csrc/bindings.cpp:15-30,147-183). No kernel runs here."""
import random
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
BF, F32, I32 = torch.bfloat16, torch.float32, torch.int32
D = 256
INVALID = 1  # hipErrorInvalidValue


def declared_symbols():
    """Every qe_* entry point declared in include/*.h (comments stripped)."""
    syms = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        syms |= set(re.findall(r"\b(qe_\w+)\s*\(", text))
    return sorted(syms)


def test_header_declares_the_path():
    syms = declared_symbols()
    for s in ("qe_attn_prep", "qe_attn_decode", "qe_attn_decode_partials",
              "qe_attn_decode_combine", "qe_attn_split_size", "qe_attn_version", "qe_gemv_bf16",
              "qe_gemv_kparts", "qe_gemv_tile_rows", "qe_hbm_read_probe"):
        assert s in syms


def test_library_exports_every_declared_symbol(capi):
    lib = capi.load()
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(capi.SIGNATURES) == set(declared_symbols())


def test_version_and_split_size(capi):
    assert "gfx950" in capi.version()
    assert capi.split_size(4096, 16) == 256          # the reference engine's defaults
    assert capi.split_size(16384, 64) == 256
    assert capi.split_size(1000, 3) == 352           # ceil(1000/3) = 334 -> multiple of 32
    assert capi.split_size(10, 100) == 32            # never below one 32-position tile
    assert capi.split_size(0, 4) == 0 and capi.split_size(8, 0) == 0
    for L in (1, 31, 32, 33, 4097, 131072):    # slice size of a row attending L positions
        for ns in (1, 7, 16, 512):
            ch = capi.split_size(L, ns)
            assert ch % 32 == 0 and ch * ns >= L and (ch == 32 or ch - 32 < -(-L // ns))
    assert capi.split_size(1 << 23, 4) == 0      # beyond the kernels' length range


def test_split_size_multiply_shift_is_exact(capi):
    """The kernels divide by NS with a host-computed multiply and shift; qe_attn_split_size runs
    the same inline arithmetic. Compare it with exact integer division at the edges of the
    length range, at multiples of NS and their neighbours, and at seeded random points."""
    rng = random.Random(5)
    ns_list = [1, 2, 3, 5, 7, 16, 31, 64, 100, 127, 128, 129, 1000, 4095, 65537, (1 << 23) - 1,
               (1 << 31) - 1] + [rng.randrange(1, 1 << 20) for _ in range(40)]
    top = (1 << 23) - 1
    for ns in ns_list:
        Ls = {1, 2, top, top - 1, ns, ns + 1, 2 * ns, 2 * ns + 1, 32 * ns, 32 * ns + 1}
        Ls |= {rng.randrange(1, top + 1) for _ in range(60)}
        for L in sorted(x for x in Ls if 1 <= x <= top):
            want = max(32, -(-(-(-L // ns)) // 32) * 32)
            assert capi.split_size(L, ns) == want, (L, ns)


# Fake 16-byte aligned addresses: the C ABI validates before touching them.
A = 1 << 20


@pytest.mark.parametrize("kw,why", [
    (dict(n=0), "no rows"), (dict(n=65536), "more rows than the combine's grid"),
    (dict(hq=25), "Hq % Hkv"), (dict(ns=0), "no splits"), (dict(max_len=0), "empty cache"),
    (dict(max_len=1 << 23), "cache beyond 32-bit buffer offsets"),
    (dict(q=A + 8), "unaligned q"), (dict(kc=A + 2), "unaligned kc"),
])
def test_capi_decode_rejects(capi, kw, why):
    a = dict(q=A, kc=A, vc=A, pos=A, qg=A, ldp=24 * 512, part_o=A, part_ml=A, out=A,
             ldo=24 * D, n=1, hq=24, hkv=4, max_len=4096, ns=16)
    a.update(kw)
    r = capi.load().qe_attn_decode(a["q"], a["kc"], a["vc"], a["pos"], a["qg"], a["ldp"],
                                   a["part_o"], a["part_ml"], a["out"], a["ldo"], a["n"], a["hq"],
                                   a["hkv"], a["max_len"], a["ns"], 1.0 / 16, None)
    assert r == INVALID, why


@pytest.mark.parametrize("max_len", [(1 << 23) - 64, (1 << 23) - 1, 0])
def test_capi_stream_probes_reject_offsets_past_32_bits(capi, max_len):
    """The measurement probes step 32-bit byte offsets up to 64 rows past the cache end: cache
    lengths where that could wrap, (max_len + 64) * 512 >= 2^32, are rejected before any launch."""
    lib = capi.load()
    assert lib.qe_kv_stream_probe(A, A, A, 4, max_len, 16, A, None) == INVALID
    assert lib.qe_kv_stream_sweep(A, A, A, 4, max_len, 64, 8, A, None) == INVALID


@pytest.mark.parametrize("kw,why", [(dict(gph=0), "no workgroups"), (dict(gph=65536), "grid"),
                                    (dict(depth=5), "depth"), (dict(hkv=0), "no heads"),
                                    (dict(sink=None), "null sink")])
def test_capi_stream_sweep_rejects(capi, kw, why):
    a = dict(gph=64, depth=8, hkv=4, sink=A)
    a.update(kw)
    assert capi.load().qe_kv_stream_sweep(A, A, A, a["hkv"], 4096, a["gph"], a["depth"],
                                          a["sink"], None) == INVALID, why


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("kw,why", [
    (dict(T=0), "no rows"), (dict(hq=25), "Hq % Hkv"), (dict(hkv=0), "no kv heads"),
    (dict(max_len=0), "empty cache"), (dict(pos=None), "null pos"), (dict(q=A + 8), "q unaligned"),
    (dict(ldp=12), "qg row stride not a multiple of 8"), (dict(max_len=1 << 23), "32-bit offsets"),
])
def test_capi_prefill_rejects(capi, fp8, kw, why):
    """qe_attn_prefill / qe_attn_prefill_fp8 reject out-of-range arguments before any launch."""
    a = dict(q=A, kc=A, vc=A, pos=A, qg=A, ldp=48 * D, out=A, ldo=24 * D, T=16, hq=24, hkv=4,
             max_len=4096)
    a.update(kw)
    args = (a["q"], a["kc"], a["vc"], a["pos"], a["qg"], a["ldp"], a["out"], a["ldo"], a["T"],
            a["hq"], a["hkv"], a["max_len"], 1.0 / 16)
    lib = capi.load()
    r = lib.qe_attn_prefill_fp8(*args, 1.0, 1.0, None) if fp8 else lib.qe_attn_prefill(*args, None)
    assert r == INVALID, why


BAD_SCALES = [(0.0, 1.0), (1.0, -1.0), (float("inf"), 1.0), (1.0, float("nan")),
              (1e-39, 1.0), (1.0, 1e-45)]  # the last two: subnormal, 1/scale overflows to inf


@pytest.mark.parametrize("ks,vs", BAD_SCALES)
def test_capi_fp8_ops_reject_scales(capi, ks, vs):
    """Every fp8-cache entry point rejects scales that are not normal finite fp32 values."""
    lib = capi.load()
    assert lib.qe_attn_prefill_fp8(A, A, A, A, A, 48 * D, A, 24 * D, 16, 24, 4, 4096, 1.0 / 16,
                                   ks, vs, None) == INVALID
    assert lib.qe_attn_prep_fp8(A, A, A, 48 * D + 2048, A, A, A, A, A, A, A, 1, 24, 4, 4096, 64,
                                1e-6, ks, vs, None) == INVALID
    assert lib.qe_attn_decode_fp8(A, A, A, A, A, 48 * D, A, A, A, 24 * D, 1, 24, 4, 4096, 16,
                                  1.0 / 16, ks, vs, None) == INVALID
    if not 1.17549435e-38 <= ks <= 3.4028235e38:  # the partials take k_scale only
        assert lib.qe_attn_decode_fp8_partials(A, A, A, A, A, A, 1, 24, 4, 4096, 16, 1.0 / 16, ks,
                                               None) == INVALID


@pytest.mark.parametrize("ks,vs", BAD_SCALES)
def test_fp8_ops_contract_rejects_scales(native, ks, vs):
    with pytest.raises(RuntimeError, match="not subnormal"):
        native._check_kv_scales(ks, vs)


def test_fp8_ops_contract_accepts_normal_scales(native):
    for ks, vs in ((1.0 / 16, 1.0 / 16), (1.17549435e-38, 3.0e38), (448.0, 1e-3)):
        native._check_kv_scales(ks, vs)


@pytest.mark.parametrize("kw,why", [
    (dict(n=0), "no rows"), (dict(rd=3), "odd rotary dims"), (dict(rd=258), "rd > 256"),
    (dict(max_len=0), "empty cache"), (dict(hkv=0), "no kv heads"), (dict(qg=None), "null"),
])
def test_capi_prep_rejects(capi, kw, why):
    a = dict(qg=A, k=A, v=A, ldp=8, qnw=A, knw=A, inv=A, pos=A, q_out=A, kc=A, vc=A, n=1, hq=24,
             hkv=4, max_len=4096, rd=64)
    a.update(kw)
    r = capi.load().qe_attn_prep(a["qg"], a["k"], a["v"], a["ldp"], a["qnw"], a["knw"], a["inv"],
                                 a["pos"], a["q_out"], a["kc"], a["vc"], a["n"], a["hq"], a["hkv"],
                                 a["max_len"], a["rd"], 1e-6, None)
    assert r == INVALID, why


@pytest.mark.parametrize("kw,why", [
    (dict(n=0), "no rows"), (dict(n=65536), "more than 65535 rows"),
    (dict(rd=3), "odd rotary dims"), (dict(hq=25), "Hq % Hkv"), (dict(ns=0), "no splits"),
    (dict(q_out=A + 8), "unaligned q_out"),
    (dict(qg=None), "null qg"), (dict(out=None), "null out"),
    (dict(max_len=1 << 23), "cache beyond 32-bit buffer offsets"),
])
def test_capi_prep_decode_rejects(capi, kw, why):
    a = dict(qg=A, k=A, v=A, ldp=24 * 512 + 2048, qnw=A, knw=A, inv=A, pos=A, q_out=A, kc=A,
             vc=A, part_o=A, part_ml=A, out=A, ldo=24 * D, n=1, hq=24, hkv=4, max_len=4096, rd=64,
             ns=16)
    a.update(kw)
    r = capi.load().qe_attn_prep_decode(
        a["qg"], a["k"], a["v"], a["ldp"], a["qnw"], a["knw"], a["inv"], a["pos"], a["q_out"],
        a["kc"], a["vc"], a["part_o"], a["part_ml"], a["out"], a["ldo"], a["n"], a["hq"],
        a["hkv"], a["max_len"], a["rd"], a["ns"], 1.0 / 16, 1e-6, None)
    assert r == INVALID, why


def test_pdl_switches_are_noops(native):
    native.set_pdl_trigger(True)
    native.set_pdl_launch(False)


# ------------------------------------------------------------------ torch-level contract (CPU)
def decode_args(n=2, hq=24, hkv=4, max_len=64, ns=4, ldp_pad=8):
    q = torch.zeros(n, hq * D, dtype=BF)
    kc = torch.zeros(hkv, max_len, D, dtype=BF)
    vc = torch.zeros_like(kc)
    pos = torch.zeros(1, dtype=I32)
    qg = torch.zeros(n, hq * 2 * D + ldp_pad, dtype=BF)[:, : hq * 2 * D]
    po = torch.zeros(max(8, n), hq, ns, D, dtype=F32)
    pml = torch.zeros(max(8, n), hq, ns, 2, dtype=F32)
    out = torch.zeros(n, hq * D, dtype=BF)
    return dict(q=q, kc=kc, vc=vc, pos=pos, qg=qg, part_o=po, part_ml=pml, out=out)


def check_decode(C, a):
    return C._check_attn_decode(a["q"], a["kc"], a["vc"], a["pos"], a["qg"], a["part_o"],
                                a["part_ml"], a["out"])


def test_decode_contract_accepts_engine_layout(native):
    n, hq, hkv, max_len, ns, ldp, ldo = check_decode(native, decode_args())
    assert (n, hq, hkv, max_len, ns) == (2, 24, 4, 64, 4)
    assert ldp == 24 * 2 * D + 8 and ldo == 24 * D
    one_row = decode_args(n=1)
    one_row["q"], one_row["out"] = one_row["q"][0], one_row["out"][0]   # 1-D counts as one row
    one_row["qg"] = one_row["qg"][0]
    assert check_decode(native, one_row)[0] == 1


def _mut(**changes):
    def f(a):
        a.update({k: v(a) for k, v in changes.items()})
        return a
    return f


@pytest.mark.parametrize("mutate,msg", [
    (_mut(q=lambda a: a["q"].float()), "wrong device/dtype"),
    (_mut(kc=lambda a: a["kc"].float()), "wrong dtype"),
    (_mut(part_o=lambda a: a["part_o"].to(BF)), "wrong dtype"),
    (_mut(pos=lambda a: a["pos"].long()), "int32"),
    (_mut(kc=lambda a: a["kc"].transpose(0, 1)), "contiguous"),
    (_mut(q=lambda a: torch.zeros(2, 24 * D + 8, dtype=BF)[:, : 24 * D]), "contiguous"),
    (_mut(out=lambda a: torch.zeros(3, 24 * D, dtype=BF)), "rows must agree"),
    (_mut(kc=lambda a: torch.zeros(5, 64, D, dtype=BF), vc=lambda a: torch.zeros(5, 64, D, dtype=BF)),
     "Hq % Hkv"),
    (_mut(part_o=lambda a: torch.zeros(1, 24, 4, D)), "part_o"),
    (_mut(part_o=lambda a: torch.zeros(8, 24, 4, 128)), "part_o"),
    (_mut(part_ml=lambda a: torch.zeros(8, 24, 3, 2)), "part_ml"),
    (_mut(qg=lambda a: torch.zeros(2, 24 * D, dtype=BF)), "qg width"),
    (_mut(vc=lambda a: torch.zeros(4, 32, D, dtype=BF)), "equal sizes"),
    (_mut(kc=lambda a: torch.zeros(4, 64, 128, dtype=BF), vc=lambda a: torch.zeros(4, 64, 128, dtype=BF)),
     "256"),
    (_mut(q=lambda a: torch.zeros(2, 24 * D + 8, dtype=BF)), "q width must be Hq"),
])
def test_decode_contract_rejects(native, mutate, msg):
    a = mutate(decode_args())
    with pytest.raises(RuntimeError, match=msg):
        check_decode(native, a)


def test_decode_contract_row_limits(native):
    """Rows are bounded only by part_o.size(0) (and the combine's 65535), any group size is
    accepted, as in the reference (csrc/bindings.cpp:176-179): wider calls run as several
    partials launches."""
    assert check_decode(native, decode_args(n=9))[0] == 9
    assert check_decode(native, decode_args(n=8, hq=32, hkv=2))[:3] == [8, 32, 2]  # 128 columns
    assert check_decode(native, decode_args(n=1, hq=130, hkv=1))[:3] == [1, 130, 1]
    with pytest.raises(RuntimeError, match="1..65535 rows"):
        a = decode_args(n=1, hq=1, hkv=1)
        a["q"], a["out"] = torch.empty(65536, D, dtype=BF), torch.empty(65536, D, dtype=BF)
        a["qg"] = torch.empty(65536, 2 * D, dtype=BF)
        a["part_o"] = torch.empty(65536, 1, 4, D, dtype=F32)
        a["part_ml"] = torch.empty(65536, 1, 4, 2, dtype=F32)
        check_decode(native, a)
    with pytest.raises(RuntimeError, match="part_o"):
        a = decode_args(n=9)
        a["part_o"], a["part_ml"] = a["part_o"][:8], a["part_ml"][:8]
        check_decode(native, a)


def test_decode_requires_gpu_tensors(native):
    a = decode_args()
    with pytest.raises(RuntimeError, match="device"):
        native.attn_decode(a["q"], a["kc"], a["vc"], a["pos"], a["qg"], a["part_o"], a["part_ml"],
                           a["out"])


def prep_args(n=2, hq=24, hkv=4, max_len=64, rd=64, pad=8):
    w = hq * 2 * D + 2 * hkv * D
    proj = torch.zeros(n, w + pad, dtype=BF)
    return dict(qg=proj[:, : hq * 2 * D], k=proj[:, hq * 2 * D: hq * 2 * D + hkv * D],
                v=proj[:, hq * 2 * D + hkv * D: w], qnw=torch.zeros(D, dtype=BF),
                knw=torch.zeros(D, dtype=BF), inv_freq=torch.zeros(rd // 2, dtype=F32),
                pos=torch.zeros(1, dtype=I32), q_out=torch.zeros(n, hq * D, dtype=BF),
                kc=torch.zeros(hkv, max_len, D, dtype=BF), vc=torch.zeros(hkv, max_len, D, dtype=BF))


def check_prep(C, a):
    return C._check_attn_prep(a["qg"], a["k"], a["v"], a["qnw"], a["knw"], a["inv_freq"],
                              a["pos"], a["q_out"], a["kc"], a["vc"])


def test_prep_contract_accepts_engine_layout(native):
    n, hq, hkv, max_len, rd, ldp = check_prep(native, prep_args())
    assert (n, hq, hkv, max_len, rd) == (2, 24, 4, 64, 64)
    assert ldp == 24 * 2 * D + 2 * 4 * D + 8


@pytest.mark.parametrize("mutate,msg", [
    (_mut(k=lambda a: torch.zeros(2, 4 * D, dtype=BF)), "share a row stride"),
    (_mut(inv_freq=lambda a: torch.zeros(32, dtype=BF)), "wrong dtype"),
    (_mut(qnw=lambda a: torch.zeros(128, dtype=BF)), "256 elements"),
    (_mut(kc=lambda a: torch.zeros(4, 64, 128, dtype=BF)), "head_dim 256"),
    (_mut(vc=lambda a: torch.zeros(4, 65, D, dtype=BF)), "vc must match"),
    (_mut(inv_freq=lambda a: torch.zeros(129, dtype=F32)), "<= 256"),
    (_mut(q_out=lambda a: torch.zeros(2, 25 * D, dtype=BF)), "row widths"),
    (_mut(q_out=lambda a: torch.zeros(2, 24 * D + 8, dtype=BF)), "q_out width must be Hq"),
])
def test_prep_contract_rejects(native, mutate, msg):
    with pytest.raises(RuntimeError, match=msg):
        check_prep(native, mutate(prep_args()))


def prefill_args(T=16, hq=24, hkv=4, max_len=64, kv8=False, pad=8):
    kdt = torch.float8_e4m3fn if kv8 else BF
    return dict(q=torch.zeros(T, hq * D, dtype=BF), kc=torch.zeros(hkv, max_len, D, dtype=kdt),
                vc=torch.zeros(hkv, max_len, D, dtype=kdt), pos=torch.zeros(1, dtype=I32),
                qg=torch.zeros(T, hq * 2 * D + pad, dtype=BF)[:, : hq * 2 * D],
                out=torch.zeros(T, hq * D, dtype=BF))


def check_prefill(C, a, kv8=False):
    return C._check_attn_prefill(a["q"], a["kc"], a["vc"], a["pos"], a["qg"], a["out"], kv8)


@pytest.mark.parametrize("kv8", [False, True])
def test_prefill_contract(native, kv8):
    T, hq, hkv, max_len, ldp, ldo = check_prefill(native, prefill_args(kv8=kv8), kv8)
    assert (T, hq, hkv, max_len, ldp, ldo) == (16, 24, 4, 64, 24 * 2 * D + 8, 24 * D)
    for mutate, msg in [
            (_mut(q=lambda a: torch.zeros(16, 24 * D + 8, dtype=BF)), "q width must be Hq"),
            (_mut(q=lambda a: torch.zeros(16, 24 * D + 8, dtype=BF)[:, : 24 * D]), "contiguous"),
            (_mut(out=lambda a: torch.zeros(15, 24 * D, dtype=BF)), "rows must agree"),
            (_mut(qg=lambda a: torch.zeros(16, 24 * D, dtype=BF)), "qg width"),
            (_mut(vc=lambda a: a["vc"][:, :32].contiguous()), "equal sizes")]:
        with pytest.raises(RuntimeError, match=msg):
            check_prefill(native, mutate(prefill_args(kv8=kv8)), kv8)


def test_prep_contract_row_limit(native):
    with pytest.raises(RuntimeError, match="1..8 rows"):
        check_prep(native, prep_args(n=9))


def test_prep_decode_contract(native):
    """attn_prep_decode validates as attn_prep (on qg, k, v, ..., q_out, kc, vc) and as
    attn_decode (with q_out as q) together."""
    C = native
    n, hq, hkv, max_len, ns = 3, 24, 4, 64, 4
    a = decode_args(n=n, hq=hq, hkv=hkv, max_len=max_len, ns=ns)
    proj = torch.zeros(n, hq * 2 * D + 2 * hkv * D + 8, dtype=BF)
    qg, k, v = (proj[:, : hq * 2 * D], proj[:, hq * 2 * D: hq * 2 * D + hkv * D],
                proj[:, hq * 2 * D + hkv * D: hq * 2 * D + 2 * hkv * D])
    qnw, knw, inv = torch.zeros(D, dtype=BF), torch.zeros(D, dtype=BF), torch.zeros(32, dtype=F32)
    res = C._check_attn_prep_decode(qg, k, v, qnw, knw, inv, a["pos"], a["q"], a["kc"], a["vc"],
                                    a["part_o"], a["part_ml"], a["out"])
    assert list(res[:5]) == [n, hq, hkv, max_len, 64] and res[6] == ns
    with pytest.raises(RuntimeError, match="part_o"):
        C._check_attn_prep_decode(qg, k, v, qnw, knw, inv, a["pos"], a["q"], a["kc"], a["vc"],
                                  a["part_o"][:, :, :, :128], a["part_ml"], a["out"])
    with pytest.raises(RuntimeError, match="rows"):
        C._check_attn_prep_decode(qg[:2], k[:2], v[:2], qnw, knw, inv, a["pos"], a["q"][:2],
                                  a["kc"], a["vc"], a["part_o"], a["part_ml"], a["out"])


# ------------------------------------------------------------------ gemv_bf16 (basic.cu:99-155)
@pytest.mark.parametrize("kw,why", [
    (dict(nr=0), "no rows"), (dict(nr=9), "more than 8 rows"), (dict(K=12), "K % 8"),
    (dict(K=0), "empty rows"), (dict(N=0), "no outputs"), (dict(W=A + 8), "unaligned W"),
    (dict(x=A + 2), "unaligned x"), (dict(ldx=5112), "ldx < K"), (dict(ldx=5124), "ldx % 8"),
    (dict(ldo=100), "ldo < N"), (dict(out=None), "null out"),
    (dict(K=1 << 27), "tile beyond 32-bit buffer offsets"),
    (dict(nr=8, ldx=1 << 29), "activation rows beyond 32-bit buffer offsets"),
])
def test_capi_gemv_rejects(capi, kw, why):
    a = dict(W=A, x=A, out=A, nr=1, N=14336, K=5120, ldx=5120, ldo=14336)
    a.update(kw)
    r = capi.load().qe_gemv_bf16(a["W"], a["x"], a["out"], a["nr"], a["N"], a["K"], a["ldx"],
                                 a["ldo"], None)
    assert r == INVALID, why


def test_gemv_kparts():
    """k-parts per 16-row tile: more for small N, never below 8 MFMA k-steps per part, and a
    function of (N, K) only (so every row count reduces in the same order)."""
    import qengine_amd.capi as capi
    assert capi.gemv_kparts(248320, 5120) == 1      # lm_head: 15,520 row tiles
    assert capi.gemv_kparts(14336, 5120) == 4       # attention in_proj: 896 tiles
    assert capi.gemv_kparts(5120, 6144) == 4        # o_proj: 320 tiles
    assert capi.gemv_kparts(40000, 5120) == 2       # 2,500 tiles
    assert capi.gemv_kparts(5120, 768) == 1         # 3 blocks of 256 k: parts keep >= 2 blocks
    assert capi.gemv_kparts(5120, 1024) == 2
    assert capi.gemv_kparts(7, 64) == 1
    assert capi.gemv_kparts(0, 64) == 0


def test_gemv_tile_rows():
    """Rows per W tile: 16 unless a one-tile-per-workgroup grid of at most 4 workgroups per CU
    leaves the last round part-empty; then the height that fills it best (no GPU here: 256 CUs
    assumed, MI355X's count)."""
    import qengine_amd.capi as capi
    assert capi.gemv_tile_rows(5120, 6144) == 10     # o_proj: 320 -> 512 workgroups
    assert capi.gemv_tile_rows(14336, 5120) == 14    # in_proj: 896 -> 1024 workgroups
    assert capi.gemv_tile_rows(4096, 6144) == 16     # 256 workgroups already fill the CUs
    assert capi.gemv_tile_rows(248320, 5120) == 16   # lm_head: 1 k-part, 16 rounds
    assert capi.gemv_tile_rows(40000, 5120) == 16    # 2 k-parts
    assert capi.gemv_tile_rows(16400, 5120) == 16    # 1,025 tiles: more than 4 per CU
    assert capi.gemv_tile_rows(1000, 1024) == 16     # 2 k-parts (4 blocks of 256 k)
    assert capi.gemv_tile_rows(1000, 2048) == 10     # 63 -> 100 workgroups
    assert capi.gemv_tile_rows(7, 64) == 16
    assert capi.gemv_tile_rows(0, 64) == 0
    assert capi.gemv_tile_rows(64, 0) == 0


def test_gemv_contract(native):
    """gemv_bf16 accepts the engine's layout (weights [N, K], a row view of the activations in a
    wider buffer, a row view of the output) and rejects what the reference rejects."""
    C = native
    W = torch.zeros(1000, 1024, dtype=BF)
    xb = torch.zeros(5, 1024 + 16, dtype=BF)
    ob = torch.zeros(5, 1000 + 8, dtype=BF)
    assert list(C._check_gemv_bf16(W, xb[:, :1024], ob[:, :1000])) == [5, 1000, 1024, 1040, 1008]
    assert list(C._check_gemv_bf16(W, xb[0, :1024], ob[0, :1000]))[:3] == [1, 1000, 1024]
    with pytest.raises(RuntimeError, match="1..8 rows"):
        C._check_gemv_bf16(W, torch.zeros(9, 1024, dtype=BF), torch.zeros(9, 1000, dtype=BF))
    with pytest.raises(RuntimeError, match="multiple of 8"):
        C._check_gemv_bf16(torch.zeros(8, 12, dtype=BF), torch.zeros(1, 12, dtype=BF),
                           torch.zeros(1, 8, dtype=BF))
    with pytest.raises(RuntimeError, match="gemv_bf16"):
        C._check_gemv_bf16(W, xb[:, :1024], ob[:4, :1000])
    with pytest.raises(RuntimeError, match="contiguous"):
        C._check_gemv_bf16(W.t(), xb[:, :1000], ob[:, :1000])
    with pytest.raises(RuntimeError, match="wrong"):
        C._check_gemv_bf16(W.float(), xb[:, :1024], ob[:, :1000])
    with pytest.raises(RuntimeError, match="aligned"):
        C._check_gemv_bf16(W, xb[:, 1:1025], ob[:, :1000])
    with pytest.raises(RuntimeError, match="GPU"):
        C.gemv_bf16(W, xb[:, :1024], ob[:, :1000])


# ------------------------------------------------------------------ the rest of the step (basic.cu)
@pytest.mark.parametrize("fn,args,why", [
    ("qe_embed", (A, A, A, 0, 64, 10, 64, None), "no rows"),
    ("qe_embed", (A, A, A, 1, 64, 10, 32, None), "ldo < H"),
    ("qe_embed", (None, A, A, 1, 64, 10, 64, None), "null table"),
    ("qe_rmsnorm1p", (A, None, A, A, 0, 64, 64, 0, 64, 1e-6, None), "no rows"),
    ("qe_rmsnorm1p", (A, A, A, A, 1, 64, 64, 32, 64, 1e-6, None), "ldd < H with delta"),
    ("qe_swiglu", (A, A, 1, 64, 100, 64, None), "ldg < 2I"),
    ("qe_argmax", (A, 1, 100, 50, A, A, 4, A, None, None), "ldx < n"),
    ("qe_argmax", (A, 1, 100, 100, A, A, 0, A, None, None), "no partials"),
    ("qe_accept", (A, A, 9, A, A, A, 10, None), "more than 8 rows"),
    ("qe_accept", (A, A, 0, A, A, A, 10, None), "no rows"),
    ("qe_commit", (A, A, A, None, 2, None), "drafts missing"),
    ("qe_mtp_select", (A, A, 0, A, 64, None, 64, None, None, None), "src without dst"),
    ("qe_mtp_select", (A, A, 0, None, 0, None, 0, None, A, None), "draft0 without mtp_am"),
])
def test_capi_step_ops_reject(capi, fn, args, why):
    assert getattr(capi.load(), fn)(*args) == INVALID, why


def test_capi_l2_controls_succeed_without_a_gpu(capi):
    lib = capi.load()
    assert lib.qe_l2_persist_limit(60 << 20) == 0
    assert lib.qe_stream_access_window(0, 0, 0.0, None) == 0


def test_step_ops_contract(native):
    """The reference's checks for embed / rmsnorm1p / argmax / accept / commit
    (csrc/bindings.cpp:33-55,68-124), exercised without a GPU."""
    C = native
    tab = torch.zeros(100, 64, dtype=BF)
    ob = torch.zeros(3, 72, dtype=BF)
    assert list(C._check_embed(tab, torch.zeros(3, dtype=I32), ob[:, :64])) == [3, 64, 100, 72]
    with pytest.raises(RuntimeError, match="tok"):
        C._check_embed(tab, torch.zeros(3, dtype=torch.int64), ob[:, :64])
    with pytest.raises(RuntimeError, match="embed"):
        C._check_embed(tab, torch.zeros(2, dtype=I32), ob[:, :64])
    x = torch.zeros(4, 5120, dtype=BF)
    w = torch.zeros(5120, dtype=BF)
    assert list(C._check_rmsnorm1p(x, None, w, x)) == [4, 5120, 5120, 0, 5120]
    assert list(C._check_rmsnorm1p(x, x, w, x))[3] == 5120
    with pytest.raises(RuntimeError, match="rmsnorm1p"):
        C._check_rmsnorm1p(x, None, w[:100], x)
    with pytest.raises(RuntimeError, match="delta"):
        C._check_rmsnorm1p(x, x[:2], w, x)
    lg = torch.zeros(5, 1000, dtype=BF)
    assert list(C._check_argmax(lg, torch.zeros(5 * 256), torch.zeros(5 * 256, dtype=I32),
                                torch.zeros(5, dtype=I32))) == [5, 1000, 1000, 256]
    with pytest.raises(RuntimeError, match="argmax"):
        C._check_argmax(lg, torch.zeros(5 * 256), torch.zeros(5 * 128, dtype=I32),
                        torch.zeros(5, dtype=I32))
    with pytest.raises(RuntimeError, match="idmap"):
        C._check_argmax(lg, torch.zeros(5), torch.zeros(5, dtype=I32), torch.zeros(5, dtype=I32),
                        torch.zeros(999, dtype=I32))
    ints = lambda k: torch.zeros(k, dtype=I32)  # noqa: E731
    C._check_accept(ints(9), ints(8), 8, ints(24), ints(8), ints(100))
    with pytest.raises(RuntimeError, match="accept"):
        C._check_accept(ints(8), ints(8), 8, ints(24), ints(8), ints(100))   # in_tok must hold n+1
    with pytest.raises(RuntimeError, match="accept"):
        C._check_accept(ints(9), ints(8), 8, ints(16), ints(8), ints(100))   # ctl >= 24
    C._check_commit(ints(24), ints(8), ints(8), ints(7), 7)
    with pytest.raises(RuntimeError, match="commit"):
        C._check_commit(ints(24), ints(7), ints(8), ints(7), 7)


# ------------------------------------------------------------------ Gated DeltaNet step (gdn.cu)
def _gdn_args(**kw):
    """qe_gdn_step_n arguments for hk=16, hv=48 (C = 10240) with fake but aligned pointers."""
    a = dict(qkv=A, z=A, b=A, a=A, ldp=16504, ring=A, conv_w=A, A_log=A, dt_bias=A, norm_w=A,
             S=A, st_k=A, st_v=A, st_g=A, ctl=A, out=A, ldo=6144, n=1, Hk=16, Hv=48, eps=1e-6,
             stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,why", [
    (dict(n=0), "no rows"), (dict(n=9), "more than 8 rows"), (dict(Hv=40), "Hv % Hk != 0"),
    (dict(Hk=0), "no qk heads"), (dict(ldp=10000), "ldp < C"), (dict(ldo=6000), "ldo < Hv*128"),
    (dict(S=A + 4), "S not 16-byte aligned"), (dict(st_g=A + 4), "st_g not 8-byte aligned"),
    (dict(conv_w=A + 2), "conv_w not 8-byte aligned"), (dict(ctl=None), "null ctl"),
    (dict(Hk=1, Hv=65536, ldp=1 << 40, ldo=1 << 40), "more value heads than grid blocks"),
])
def test_capi_gdn_rejects(capi, kw, why):
    assert capi.load().qe_gdn_step_n(*_gdn_args(**kw)) == INVALID, why


def _gdn_tensors(hk=16, hv=48, n=3, pad=24):
    Cd = 2 * hk * 128 + hv * 128
    w = Cd + hv * 128 + 2 * hv
    pr = torch.zeros(n, w + pad, dtype=BF)
    c1 = Cd + hv * 128
    return dict(qkv=pr[:, :Cd], z=pr[:, Cd:c1], b=pr[:, c1:c1 + hv], a=pr[:, c1 + hv:w],
                ring=torch.zeros(16, Cd, dtype=BF), conv_w=torch.zeros(Cd, 1, 4, dtype=BF),
                A_log=torch.zeros(hv, dtype=BF), dt_bias=torch.zeros(hv, dtype=BF),
                norm_w=torch.zeros(128, dtype=BF), S=torch.zeros(hv, 128, 128),
                st_k=torch.zeros(8, hv, 128), st_v=torch.zeros(8, hv, 128),
                st_g=torch.zeros(8, hv, 2), ctl=torch.zeros(8, dtype=I32),
                out=torch.zeros(n, hv * 128, dtype=BF), Hk=hk)


def test_gdn_contract(native):
    """The reference's checks for gdn_step_n (csrc/bindings.cpp:118-145) without a GPU."""
    C = native
    t = _gdn_tensors()
    assert list(C._check_gdn_step_n(**t)) == [3, 48, t["qkv"].stride(0), 6144]

    def bad(msg, **kw):
        u = dict(t)
        u.update(kw)
        with pytest.raises(RuntimeError, match=msg):
            C._check_gdn_step_n(**u)

    bad("share a row stride", z=torch.zeros(3, 6144, dtype=BF))
    bad("1..8 rows", out=torch.zeros(2, 6144, dtype=BF))
    t9 = _gdn_tensors(n=9)
    with pytest.raises(RuntimeError, match="1..8 rows"):
        C._check_gdn_step_n(**t9)
    bad("dk = dv = 128", S=torch.zeros(48, 64, 128))
    bad("multiple of Hk", Hk=5)
    bad("ring", ring=torch.zeros(15, 10240, dtype=BF))
    bad("conv_w", conv_w=torch.zeros(10240, 3, dtype=BF))
    bad("Hv\\*128 wide", out=torch.zeros(3, 6000, dtype=BF))
    bad("A_log", norm_w=torch.zeros(64, dtype=BF))
    bad("st_k", st_g=torch.zeros(8, 48, 1))
    bad("wrong dtype", S=torch.zeros(48, 128, 128, dtype=torch.float64))
    bad("ctl", ctl=torch.zeros(1, dtype=I32))
    with pytest.raises(RuntimeError, match="device"):
        C.gdn_step_n(**t, eps=1e-6)
    C.set_gdn_phases(True)
    C.set_gdn_early(True)


def test_default_splits_policy():
    """Split count: 13/16 of the CUs in workgroups for a bf16 cache, one workgroup per CU for fp8,
    never a slice shorter than 32 positions."""
    import qengine_amd as qa
    assert qa.default_splits(16384, 4, cus=256) == 52
    assert qa.default_splits(131072, 4, cus=256) == 52
    assert qa.default_splits(16384, 4, cus=256, kv8=True) == 64
    assert qa.default_splits(16384, 8, cus=256) == 26
    assert qa.default_splits(1000, 4, cus=256) == 32  # ceil(1000 / 32)
    assert qa.default_splits(64, 4, cus=256, kv8=True) == 2
    assert qa.default_splits(1, 64, cus=4) == 1
