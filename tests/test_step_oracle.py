"""CPU pins for oracle/step_oracle.py: closed forms, torch's own ops (the semantics the
reference's tests assert, tests/test_kernels.py:36-160 of qengine), and hand-worked scenarios of
the step bookkeeping (csrc/basic.cu:241-307)."""
import math

import pytest
import torch

import oracle as O

S = O.step_oracle
BF = torch.bfloat16


def test_embed_gathers_rows_and_zeroes_bad_ids():
    tab = torch.randn(7, 12).to(BF)
    out = S.embed(tab, [3, 6, 0, 7, -1], 5)
    assert torch.equal(out[0], tab[3]) and torch.equal(out[1], tab[6]) and torch.equal(out[2], tab[0])
    assert torch.equal(out[3:], torch.zeros(2, 12, dtype=BF))


def test_residual_add_is_one_bf16_rounding_and_nan_stays_in_its_row():
    g = torch.Generator().manual_seed(1)
    h = torch.randn(3, 64, generator=g).to(BF)
    d = torch.randn(3, 64, generator=g).to(BF)
    d[1, 5] = float("nan")
    w = (torch.randn(64, generator=g) * 0.3).to(BF)
    nh, y = S.residual_rmsnorm1p(h, d, w, 1e-6)
    want = (h.double() + d.double()).to(BF)  # exact sum, rounded once
    assert torch.equal(nh.nan_to_num(7.0), want.nan_to_num(7.0))
    assert torch.isnan(y[1]).all() and not torch.isnan(y[0]).any() and not torch.isnan(y[2]).any()
    assert torch.equal(S.residual_rmsnorm1p(h, None, w, 1e-6)[0], h)


def _silu64(x: float) -> float:
    if x == -math.inf:
        return math.nan
    return x / (1.0 + math.exp(-x)) if x > -700 else 0.0 * x


def test_swiglu_matches_an_fp64_model_of_the_rounding_chain():
    g = torch.Generator().manual_seed(2)
    gu = (torch.randn(2, 2 * 500, generator=g) * 4).to(BF)
    gu[0, 0] = float("-inf")
    gu[0, 1] = 0.0
    out = S.swiglu(gu)
    exact = 0
    for r in range(2):
        for i in range(500):
            gv, uv = float(gu[r, i]), float(gu[r, 500 + i])
            s = torch.tensor(_silu64(gv), dtype=torch.float64).to(BF)
            want = torch.tensor(float(s) * uv, dtype=torch.float64).to(BF)
            got = out[r, i]
            if math.isnan(float(want)):
                assert math.isnan(float(got))
                continue
            spacing = 2.0 ** (math.floor(math.log2(max(abs(float(want)), 1e-30))) - 7)
            assert abs(float(got) - float(want)) <= spacing, (r, i, float(got), float(want))
            exact += float(got) == float(want)
    assert out[0, 1] == 0.0
    assert exact >= 0.99 * 999


@pytest.mark.parametrize("n", [1, 7, 1000, 4097])
def test_argmax_is_torch_argmax(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(3, n, generator=g).to(BF)
    assert S.argmax(x).tolist() == x.argmax(-1).tolist()
    x[:] = 1.0
    assert S.argmax(x).tolist() == [0, 0, 0]
    if n > 3:
        x = torch.randn(1, n, generator=g).to(BF)
        x[0, n // 2] = 50.0
        x[0, n - 1] = 50.0
        assert int(S.argmax(x)[0]) == n // 2 == int(x.argmax())
        x[0, n - 2] = float("nan")
        assert int(S.argmax(x)[0]) == n - 2 == int(x.argmax())
        x = torch.full((1, n), float("-inf")).to(BF)
        assert int(S.argmax(x)[0]) == 0 == int(x.argmax())


def test_accept_verify_partial_match_and_commit():
    """Verify pass of 4 rows at pos 100: drafts 11, 12 match, 99 does not -> m = 2; the bonus
    token am[2] = 13 starts the next pass."""
    in_tok = [10, 11, 12, 99, -1]
    am = [11, 12, 13, 14]
    ctl = [0] * 24
    ctl[0], ctl[2] = 100, 1
    nt, log = [0] * 4, [0] * 110
    S.accept(in_tok, am, 4, ctl, nt, log)
    assert ctl[3] == 2 and ctl[4] == 1 and ctl[5] == 2 and ctl[18] == 1
    assert log[101:104] == [11, 12, 13] and log[104] == 0
    assert nt == am
    S.commit(ctl, in_tok, am, [7, 8, 9], 3)
    assert ctl[0] == 103 and ctl[1] == 3 and in_tok[:4] == [13, 7, 8, 9]


def test_accept_verify_all_and_none_and_log_edge():
    for in_tok, m in (([5, 1, 2, 3], 3), ([5, 9, 2, 3], 0)):
        ctl = [0] * 24
        ctl[0], ctl[2] = 6, 1
        nt, log = [0] * 4, [0] * 9
        S.accept(in_tok + [-1], [1, 2, 3, 4], 4, ctl, nt, log)
        assert ctl[3] == m and ctl[16 + m] == 1
        # positions 7.. get the accepted tokens; the log holds 9 entries, so at most 7 and 8
        assert log[7:9] == [1, 2][: min(m + 1, 2)] + [0] * (2 - min(m + 1, 2))


def test_accept_prefill_chunks():
    ctl = [0] * 24
    ctl[0] = 10  # mode 0: prefill
    nt, log = [0] * 3, [0] * 20
    S.accept([1, 2, 3, 4], [7, 8, 9], 3, ctl, nt, log)  # more prompt follows (in_tok[3] = 4)
    assert ctl[3] == 2 and nt == [2, 3, 4] and log == [0] * 20
    S.accept([1, 2, 3, -1], [7, 8, 9], 3, ctl, nt, log)  # last chunk: row 2 yields a new token
    assert nt == [2, 3, 9] and log[13] == 9 and ctl[4] == 0


def test_mtp_select():
    ctl = [0] * 24
    ctl[0], ctl[3] = 50, 2
    src = torch.arange(12, dtype=torch.float32).reshape(4, 3).to(BF)
    assert S.mtp_select(ctl, -1)[0] == 50
    mpos, row, d0 = S.mtp_select(ctl, 0, src, [4, 5, 6, 7])
    assert mpos == 53 and torch.equal(row, src[2]) and d0 == 6
    assert S.mtp_select(ctl, 2)[0] == 55
