"""GPU parity tests of the rest of the decode step (embed, rmsnorm1p with the fused residual,
swiglu, argmax, accept / commit / mtp_select) against the CPU oracle, with the reference's own
bars (tests/test_kernels.py:36-160 of qengine): exact copies and integer results, RMSNorm1p and
SwiGLU within one bf16 ulp, argmax equal to torch's, rows of a multi-row call bit-identical to
1-row calls."""
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
I32 = torch.int32
S = O.step_oracle


def ulp_close(a, b, ulps=1):
    a, b = a.float().cpu(), b.float().cpu()
    nan_ok = torch.isnan(a) == torch.isnan(b)
    m = torch.maximum(a.abs(), b.abs())
    spacing = torch.where(m > 0, 2.0 ** (torch.floor(torch.log2(m.clamp_min(1e-38))) - 7), 1e-38)
    ok = ((a - b).abs() <= ulps * spacing) | (a == b) | (torch.isnan(a) & torch.isnan(b))
    return bool((ok & nan_ok).all()), (a - b).abs().nan_to_num().max().item()


# ------------------------------------------------------------------------------ embed
@pytest.mark.parametrize("V,H", [(7, 8), (1000, 1024), (248320, 1024), (33, 5120), (50, 12)])
def test_embed(native, V, H):
    tab = torch.randn(V, H, device=DEV).to(BF)
    tok = torch.tensor([3 % V, V - 1, 0, V + 5, -1], dtype=I32, device=DEV)
    out = torch.empty(5, H, dtype=BF, device=DEV)
    native.embed(tab, tok, out)
    assert torch.equal(out.cpu(), S.embed(tab.cpu(), tok.cpu().tolist(), 5))


def test_embed_strided_output(native):
    tab = torch.randn(100, 64, device=DEV).to(BF)
    tok = torch.tensor([5, 99], dtype=I32, device=DEV)
    ob = torch.full((2, 72), 3.0, dtype=BF, device=DEV)
    native.embed(tab, tok, ob[:, :64])
    assert torch.equal(ob[:, :64].cpu(), S.embed(tab.cpu(), [5, 99], 2))
    assert bool((ob[:, 64:] == 3.0).all())


# ------------------------------------------------------------------------------ rmsnorm1p
@pytest.mark.parametrize("rows,H", [(1, 1024), (1, 5120), (1, 1000), (8, 256), (3, 7), (1, 127),
                                    (4, 4097), (2, 8192 + 8)])
@pytest.mark.parametrize("scale", [1.0, 1e-3, 300.0])
def test_rmsnorm1p(native, rows, H, scale):
    g = torch.Generator().manual_seed(rows * H)
    x = (torch.randn(rows, H, generator=g) * scale).to(BF)
    w = (torch.randn(H, generator=g) * 0.3).to(BF)
    out = torch.empty(rows, H, dtype=BF, device=DEV)
    native.rmsnorm1p(x.to(DEV), None, w.to(DEV), out, 1e-6)
    ok, err = ulp_close(out, O.rmsnorm1p(x, w, 1e-6))
    assert ok, err


@pytest.mark.parametrize("H", [1024, 5120, 1000])
def test_rmsnorm1p_fused_residual_and_nan(native, H):
    g = torch.Generator().manual_seed(H)
    h = torch.randn(4, H, generator=g).to(BF)
    d = torch.randn(4, H, generator=g).to(BF)
    d[2, 5] = float("nan")  # NaN stays in its row
    d[3, 0] = float("inf")
    w = torch.randn(H, generator=g).to(BF)
    h_ref, y_ref = S.residual_rmsnorm1p(h, d, w, 1e-6)
    hd = h.to(DEV)
    out = torch.empty(4, H, dtype=BF, device=DEV)
    native.rmsnorm1p(hd, d.to(DEV), w.to(DEV), out, 1e-6)
    assert torch.equal(hd.cpu().nan_to_num(9.0), h_ref.nan_to_num(9.0))  # residual add exact
    ok, err = ulp_close(out, y_ref)
    assert ok, err
    assert torch.isnan(out[2].float()).all() and not torch.isnan(out[:2].float()).any()


def test_rmsnorm1p_rows_bit_exact(native):
    H = 5120
    x = torch.randn(8, H, device=DEV).to(BF)
    w = torch.randn(H, device=DEV).to(BF)
    out = torch.empty(8, H, dtype=BF, device=DEV)
    native.rmsnorm1p(x, None, w, out, 1e-6)
    one = torch.empty(1, H, dtype=BF, device=DEV)
    for r in range(8):
        native.rmsnorm1p(x[r:r + 1].clone(), None, w, one, 1e-6)
        assert torch.equal(out[r], one[0]), r


# ------------------------------------------------------------------------------ swiglu
@pytest.mark.parametrize("I", [1, 7, 127, 3584, 17408, 4097])
def test_swiglu(native, I):
    g = torch.Generator().manual_seed(I)
    gu = (torch.randn(2 * I, generator=g) * 4).to(BF)
    if I > 1:
        gu[0] = float("-inf")
    out = torch.empty(I, dtype=BF, device=DEV)
    native.swiglu(gu.to(DEV), out)
    ok, err = ulp_close(out, S.swiglu(gu))
    assert ok, err
    gu2 = gu.to(DEV).repeat(3, 1)
    out2 = torch.empty(3, I, dtype=BF, device=DEV)
    native.swiglu(gu2, out2)
    assert torch.equal(out2.view(torch.int16), out.expand(3, I).view(torch.int16))  # NaN-safe


# ------------------------------------------------------------------------------ argmax
def _argmax(C, x, nb=256, idmap=None):
    rows = 1 if x.dim() == 1 else x.shape[0]
    out = torch.empty(rows, dtype=I32, device=DEV)
    C.argmax(x, torch.empty(rows * nb, device=DEV), torch.empty(rows * nb, dtype=I32, device=DEV),
             out, idmap)
    return out.cpu()


def test_argmax_rows(native):
    x = torch.randn(5, 248320, device=DEV).to(BF)
    assert _argmax(native, x).tolist() == S.argmax(x.cpu()).tolist() == x.argmax(-1).tolist()


@pytest.mark.parametrize("n", [1, 7, 127, 1000, 4097, 32768, 248320])
@pytest.mark.parametrize("nb", [256, 3])
def test_argmax(native, n, nb):
    x = torch.randn(n, device=DEV).to(BF)
    assert int(_argmax(native, x, nb)[0]) == int(x.argmax())
    x[:] = 1.0  # all ties -> lowest index
    assert int(_argmax(native, x, nb)[0]) == 0
    if n > 3:
        x = torch.randn(n, device=DEV).to(BF)
        x[n // 2] = 50.0
        x[n - 1] = 50.0  # tie between two maxima -> lower index
        assert int(_argmax(native, x, nb)[0]) == n // 2 == int(x.argmax())
        x[n - 2] = float("nan")  # torch: NaN is the max
        assert int(_argmax(native, x, nb)[0]) == n - 2 == int(x.argmax())
        x = torch.full((n,), float("-inf"), device=DEV).to(BF)
        assert int(_argmax(native, x, nb)[0]) == 0 == int(x.argmax())


def test_argmax_unaligned_rows_and_idmap(native):
    xb = torch.randn(3, 1001, device=DEV).to(BF)
    x = xb[:, 1:]  # rows start 2 bytes into the buffer: the scalar path
    assert _argmax(native, x, 7).tolist() == x.argmax(-1).tolist()
    idmap = torch.randperm(1000, device=DEV).to(I32)
    want = idmap[x.argmax(-1)].tolist()
    assert _argmax(native, x, 16, idmap).tolist() == want


# ------------------------------------------------------------------------------ bookkeeping
def _dev_ints(v):
    return torch.tensor(v, dtype=I32, device=DEV)


@pytest.mark.parametrize("case", ["verify_partial", "verify_all", "verify_none", "log_edge",
                                  "prefill_more", "prefill_last"])
def test_accept_commit_match_the_oracle(native, case):
    n, P, mode, log_len = 4, 100, 1, 110
    am = [11, 12, 13, 14]
    in_tok = {"verify_partial": [10, 11, 12, 99, -1], "verify_all": [10, 11, 12, 13, -1],
              "verify_none": [10, 5, 12, 13, -1], "log_edge": [10, 11, 12, 13, -1],
              "prefill_more": [1, 2, 3, 4, 5], "prefill_last": [1, 2, 3, 4, -1]}[case]
    if case == "log_edge":
        log_len = 103
    if case.startswith("prefill"):
        mode = 0
    ctl = [0] * 24
    ctl[0], ctl[2], ctl[4], ctl[5] = P, mode, 7, 9
    nt, log = [0] * n, [0] * log_len
    drafts = [21, 22, 23]
    ref_in, ref_ctl, ref_nt, ref_log = list(in_tok), list(ctl), list(nt), list(log)
    S.accept(ref_in, am, n, ref_ctl, ref_nt, ref_log)
    S.commit(ref_ctl, ref_in, am, drafts, 3)

    d_in, d_am, d_ctl = _dev_ints(in_tok), _dev_ints(am), _dev_ints(ctl)
    d_nt, d_log, d_dr = _dev_ints(nt), _dev_ints(log), _dev_ints(drafts)
    native.accept(d_in, d_am, n, d_ctl, d_nt, d_log)
    native.commit(d_ctl, d_in, d_am, d_dr, 3)
    assert d_ctl.tolist() == ref_ctl
    assert d_nt.tolist() == ref_nt and d_log.tolist() == ref_log and d_in.tolist() == ref_in


@pytest.mark.parametrize("off", [-1, 0, 2])
def test_mtp_select(native, off):
    ctl = [0] * 24
    ctl[0], ctl[3] = 40, 2
    src = torch.randn(4, 5120, device=DEV).to(BF)
    dst = torch.empty(5120, dtype=BF, device=DEV)
    mtp_am = [4, 5, 6, 7]
    mpos, d0 = _dev_ints([0]), _dev_ints([0])
    native.mtp_select(_dev_ints(ctl), mpos, off, src, dst, _dev_ints(mtp_am), d0)
    want_pos, want_row, want_d0 = S.mtp_select(ctl, off, src.cpu(), mtp_am)
    assert int(mpos) == want_pos and int(d0) == want_d0 and torch.equal(dst.cpu(), want_row)
    mpos2 = _dev_ints([0])
    native.mtp_select(_dev_ints(ctl), mpos2, off)  # position only
    assert int(mpos2) == want_pos


def test_l2_controls_are_noops(native):
    native.l2_persist_limit(60 << 20)
    native.stream_window(0, 0, 0.0)
    native.l2_persist_limit(0)


def test_step_ops_under_graph_capture(native):
    """embed -> rmsnorm1p -> swiglu -> argmax -> accept -> commit captured once and replayed
    (the device bookkeeping advances pos every replay) == the same ops run eagerly."""
    V, H, I = 1000, 512, 256
    tab = torch.randn(V, H, device=DEV).to(BF)
    w = torch.randn(H, device=DEV).to(BF)

    def state():
        ctl = torch.zeros(24, dtype=I32, device=DEV)
        ctl[2] = 1
        return dict(ctl=ctl, in_tok=_dev_ints([3, 4, 5, -1]), h=torch.empty(3, H, dtype=BF, device=DEV),
                    xn=torch.empty(3, H, dtype=BF, device=DEV), act=torch.empty(3, I, dtype=BF, device=DEV),
                    am=torch.empty(3, dtype=I32, device=DEV), nt=torch.empty(3, dtype=I32, device=DEV),
                    log=torch.zeros(64, dtype=I32, device=DEV), ws_v=torch.empty(3 * 8, device=DEV),
                    ws_i=torch.empty(3 * 8, dtype=I32, device=DEV), drafts=_dev_ints([7, 8]))

    def step(s):
        native.embed(tab, s["in_tok"], s["h"])
        native.rmsnorm1p(s["h"], None, w, s["xn"], 1e-6)
        native.swiglu(s["xn"], s["act"])
        native.argmax(s["act"], s["ws_v"], s["ws_i"], s["am"])
        native.accept(s["in_tok"], s["am"], 3, s["ctl"], s["nt"], s["log"])
        native.commit(s["ctl"], s["in_tok"], s["am"], s["drafts"], 2)

    eager, cap = state(), state()
    for _ in range(3):
        step(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    warm = state()
    with torch.cuda.stream(side):
        step(warm)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(cap)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
    for k in ("ctl", "in_tok", "log", "am", "nt"):
        assert torch.equal(cap[k], eager[k]), k
