"""Known-answer vectors (tests/golden/*.npz, written by tests/golden/make_golden.py from the
independent float64 models) against the CPU oracle and, on a GPU, against the HIP kernels.

Expected values are float64 evaluations with the reference's bf16 rounding points, so the oracle
(fp32, like the reference) and the kernels may differ from them where a value sits at a bf16
rounding boundary: prep within 1 bf16 ulp (the reference's own bar, tests/test_kernels.py:342-345
of qengine), gated outputs within 2 ulps + 2^-13 absolute (16x tighter than the reference's
2e-3), and almost all elements exact.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
BF = torch.bfloat16
D = 256


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf(a: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> bf16 tensor."""
    return torch.from_numpy((a.astype(np.uint32) << 16).view(np.float32).copy()).to(BF)


def within_ulps(a: torch.Tensor, b: torch.Tensor, ulps: int, exact_frac: float, atol: float = 0.0):
    """|a-b| <= ulps * bf16 spacing + atol everywhere, and at least exact_frac of the elements
    equal. atol covers outputs near zero, where cancellation in P.V makes a tiny absolute
    difference many ulps."""
    a, b = a.float(), b.float()
    spacing = torch.exp2(torch.floor(torch.log2(torch.maximum(a.abs(), b.abs()).clamp_min(1e-30))) - 7)
    ok = bool(((a - b).abs() <= ulps * spacing + atol).all())
    frac = (a == b).float().mean().item()
    return ok and frac >= exact_frac, (a - b).abs().max().item(), frac


PREP = ["prep_gqa6_rows3", "prep_rows_past_cache", "prep_long_position"]
DECODE = ["decode_gqa6_rows2", "decode_gqa4_rows5_clamped", "decode_mha_row1"]


def prep_inputs(z):
    hq, hkv, max_len = int(z["hq"]), int(z["hkv"]), int(z["max_len"])
    qg, k, v = bf(z["qg"]), bf(z["k"]), bf(z["v"])
    kc = torch.zeros(hkv, max_len, D, dtype=BF)
    return qg, k, v, bf(z["qnw"]), bf(z["knw"]), torch.from_numpy(z["inv_freq"]), int(z["pos"]), kc, hq, hkv


@pytest.mark.parametrize("name", PREP)
def test_oracle_prep_known_answers(name):
    z = load(name)
    qg, k, v, qnw, knw, inv, pos, kc, hq, hkv = prep_inputs(z)
    vc = kc.clone()
    q_out = O.attn_prep(qg, k, v, qnw, knw, inv, pos, kc, vc, float(z["eps"]), hq)
    ok, mx, frac = within_ulps(q_out, bf(z["q_out"]), 1, 0.99)
    assert ok, (mx, frac)
    n, max_len = qg.shape[0], kc.shape[1]
    want_k = bf(z["k_rows"])
    for t in range(n):
        if pos + t < max_len:
            ok, mx, frac = within_ulps(kc[:, pos + t], want_k[t], 1, 0.98)
            assert ok, (t, mx, frac)
            assert torch.equal(vc[:, pos + t], v[t].reshape(hkv, D))
    written = [pos + t for t in range(n) if pos + t < max_len]
    untouched = torch.ones(max_len, dtype=torch.bool)
    untouched[written] = False
    assert bool((kc[:, untouched] == 0).all()) and bool((vc[:, untouched] == 0).all())


@pytest.mark.parametrize("name", DECODE)
def test_oracle_decode_known_answers(name):
    z = load(name)
    out = O.attn_decode(bf(z["q"]), bf(z["kc"]), bf(z["vc"]), int(z["pos"]), bf(z["qg"]), int(z["hq"]))
    ok, mx, frac = within_ulps(out, bf(z["out"]), 2, 0.95, atol=2.0 ** -13)
    assert ok, (mx, frac)


# ------------------------------------------------------------------ the HIP kernels, same vectors
@pytest.mark.gpu
@pytest.mark.parametrize("name", PREP)
def test_kernel_prep_known_answers(native, name):
    z = load(name)
    qg, k, v, qnw, knw, inv, pos, kc, hq, hkv = prep_inputs(z)
    dev = "cuda"
    n = qg.shape[0]
    proj = torch.cat([qg, k, v], dim=1).to(dev)   # qg/k/v as strided views of one row buffer
    w = proj.shape[1]
    qg_d, k_d, v_d = proj[:, : hq * 2 * D], proj[:, hq * 2 * D: hq * 2 * D + hkv * D], proj[:, w - hkv * D:]
    kc_d, vc_d = kc.to(dev), kc.clone().to(dev)
    q_out = torch.empty(n, hq * D, dtype=BF, device=dev)
    native.attn_prep(qg_d, k_d, v_d, qnw.to(dev), knw.to(dev), inv.to(dev),
                     torch.tensor([pos], dtype=torch.int32, device=dev), q_out, kc_d, vc_d,
                     float(z["eps"]))
    torch.cuda.synchronize()
    ok, mx, frac = within_ulps(q_out.cpu(), bf(z["q_out"]), 1, 0.99)
    assert ok, (mx, frac)
    kc_h, vc_h = kc_d.cpu(), vc_d.cpu()
    want_k = bf(z["k_rows"])
    for t in range(n):
        if pos + t < kc.shape[1]:
            ok, mx, frac = within_ulps(kc_h[:, pos + t], want_k[t], 1, 0.98)
            assert ok, (t, mx, frac)
            assert torch.equal(vc_h[:, pos + t], v[t].reshape(hkv, D))


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
@pytest.mark.parametrize("ns", [1, 4, 16])
def test_kernel_decode_known_answers(native, name, ns):
    z = load(name)
    dev = "cuda"
    q, qg = bf(z["q"]).to(dev), bf(z["qg"]).to(dev)
    kc, vc = bf(z["kc"]).to(dev), bf(z["vc"]).to(dev)
    n, hq = q.shape[0], int(z["hq"])
    po = torch.empty(n, hq, ns, D, device=dev)
    pml = torch.empty(n, hq, ns, 2, device=dev)
    out = torch.empty(n, hq * D, dtype=BF, device=dev)
    native.attn_decode(q, kc, vc, torch.tensor([int(z["pos"])], dtype=torch.int32, device=dev),
                       qg, po, pml, out)
    torch.cuda.synchronize()
    ok, mx, frac = within_ulps(out.cpu(), bf(z["out"]), 2, 0.95, atol=2.0 ** -13)
    assert ok, (mx, frac)
