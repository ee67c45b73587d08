"""End-to-end on the GPU: a whole decode step (embed, per-layer norm + GEMV + attention + MLP,
final norm, lm_head, argmax, accept, commit) replayed as one hipGraph, and speculative verify
passes producing exactly the tokens of plain greedy decoding, whatever the drafts (the invariant
of the reference's tests/test_spec.py:57-67 and README.md:30-31). It holds because every op
computes row r of an n-row pass bit-identically to a 1-row pass. The hybrid engine adds Gated
DeltaNet layers, whose lazy rollback (staged rows replayed by the next pass) must give the same
tokens and, once replayed, the same recurrent state as plain decoding."""
import pytest
import torch

from mini_engine import MiniEngine

pytestmark = pytest.mark.gpu

PROMPT = [11, 523, 7, 1999, 64]
N_NEW = 40


@pytest.fixture(scope="module")
def engine(native):
    return MiniEngine(layers=2, hidden=1024, inter=2048, vocab=4096, max_len=128, seed=3)


@pytest.fixture(scope="module")
def plain(engine):
    toks = engine.generate_plain(PROMPT, N_NEW)
    assert len(set(toks)) > 3, toks  # a non-degenerate sequence
    return toks


def _drafter(plain, kind, k=3):
    P = len(PROMPT)

    def d(pos, last):
        out = []
        for j in range(k):
            idx = pos + 1 + j - P  # index into the generated tokens of position pos + 1 + j
            right = plain[idx] if 0 <= idx < len(plain) else 0
            if kind == "right" or (kind == "mixed" and (pos + j) % 3 != 0):
                out.append(right)
            else:
                out.append((right + 1) % 4096)
        return out
    return d


@pytest.mark.parametrize("kind", ["right", "wrong", "mixed"])
def test_spec_equals_plain(engine, plain, kind):
    toks, passes, ctl = engine.generate_spec(PROMPT, N_NEW, _drafter(plain, kind), k=3)
    assert toks == plain
    accepted = ctl[5]
    if kind == "right":
        assert passes <= (N_NEW + 2) // 4 + 1 and accepted >= 3 * (passes - 1)
    if kind == "wrong":
        assert accepted == 0 and passes == N_NEW - 1
    if kind == "mixed":
        assert 0 < accepted < 3 * passes


def test_plain_graph_replays_match_eager_passes(engine, plain):
    """The same decode run with every pass issued eagerly (no graph) gives the same tokens."""
    engine.prefill(PROMPT)
    for _ in range(N_NEW - 1):
        engine._pass(1, 0)
    torch.cuda.synchronize()
    P = len(PROMPT)
    assert engine.log[P: P + N_NEW].tolist() == plain


# ---------------------------------------------------------------- hybrid: Gated DeltaNet + attention
HYBRID = ["linear_attention", "linear_attention", "full_attention", "linear_attention"]


@pytest.fixture(scope="module")
def hybrid(native):
    """The reference model's layer pattern (three recurrent layers to one attention layer),
    small: the recurrent layers' lazy rollback is exercised inside the step graph."""
    return MiniEngine(layers=4, hidden=1024, inter=2048, vocab=4096, max_len=128, seed=5,
                      layer_types=HYBRID, hk=4, hv=8)


@pytest.fixture(scope="module")
def hybrid_plain(hybrid):
    toks = hybrid.generate_plain(PROMPT, N_NEW)
    assert len(set(toks)) > 3, toks
    return toks


@pytest.mark.parametrize("kind", ["right", "wrong", "mixed"])
def test_hybrid_spec_equals_plain(hybrid, hybrid_plain, kind):
    toks, passes, ctl = hybrid.generate_spec(PROMPT, N_NEW, _drafter(hybrid_plain, kind), k=3)
    assert toks == hybrid_plain
    if kind == "wrong":
        assert ctl[5] == 0 and passes == N_NEW - 1
    if kind == "mixed":
        assert 0 < ctl[5] < 3 * passes


def test_hybrid_state_after_spec_equals_plain(hybrid, hybrid_plain):
    """After the same tokens, speculative and plain decoding leave the same recurrent state once
    the pending rows are replayed (one more 1-row pass each), bit for bit."""
    P = len(PROMPT)
    hybrid.generate_spec(PROMPT, N_NEW, _drafter(hybrid_plain, "mixed"), k=3)
    stop = int(hybrid.ctl[0])
    states = []
    for mode in ("spec", "plain"):
        if mode == "plain":  # plain decoding to the same position
            hybrid.generate_plain(PROMPT, stop - P + 1)
        assert int(hybrid.ctl[0]) == stop
        hybrid.in_tok[0] = 7
        hybrid._pass(1, 0)  # replays every pending row into S
        torch.cuda.synchronize()
        states.append([L["S"].clone() for L in hybrid.layers if L["type"] == "linear_attention"])
        if mode == "spec":
            hybrid.reset()
    assert all(torch.equal(a, b) for a, b in zip(*states))


# ---------------------------------------------------------------- the reference's length
# tests/test_spec.py:57-67 of the reference checks spec == plain over 1,024 generated tokens for
# k = 1..4 drafts. Here 1,800 tokens on a 2,048-position cache at the default split count (52 on
# MI355X): a row attending L positions uses slices of split_size(L, 52), 32 positions up to
# L = 1,664 and 64 after, so the run crosses a change of slice size, where verify passes hold
# rows on both sides of it (one pass per size inside the kernel).
N_LONG = 1800


@pytest.fixture(scope="module")
def long_engine(native):
    return MiniEngine(layers=2, hidden=1024, inter=2048, vocab=4096, max_len=2048, seed=7)


@pytest.fixture(scope="module")
def long_plain(long_engine):
    toks = long_engine.generate_plain(PROMPT, N_LONG)
    assert len(set(toks)) > 3, toks
    return toks


def test_long_run_crosses_a_slice_size_change(long_engine):
    import qengine_amd as qa
    ns = long_engine.part_o.shape[2]
    assert ns == qa.default_splits(2048, 4)
    first, last = len(PROMPT) + 1, len(PROMPT) + N_LONG
    assert qa.split_size(first, ns) < qa.split_size(last, ns)


@pytest.mark.parametrize("k", [1, 2, 3, 4])
@pytest.mark.parametrize("kind", ["mixed", "right"])
def test_spec_equals_plain_long(long_engine, long_plain, k, kind):
    toks, passes, ctl = long_engine.generate_spec(PROMPT, N_LONG,
                                                  _drafter(long_plain, kind, k), k=k)
    assert toks == long_plain
    if kind == "mixed":
        assert 0 < ctl[5] < k * passes
    else:
        assert passes <= (N_LONG + k - 1) // (k + 1) + 2
