"""End-to-end on the GPU: a whole decode step (embed, per-layer norm + GEMV + attention + MLP,
final norm, lm_head, argmax, accept, commit) replayed as one hipGraph, and speculative verify
passes producing exactly the tokens of plain greedy decoding, whatever the drafts (the invariant
of the reference's tests/test_spec.py:57-67 and README.md:30-31). It holds because every op
computes row r of an n-row pass bit-identically to a 1-row pass."""
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


def _drafter(plain, kind):
    P = len(PROMPT)

    def d(pos, last):
        out = []
        for j in range(3):
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
