"""qe_attn_decode_noalloc (the decode with the library's own device scratch) against
qe_attn_decode with caller-owned part_o / part_ml, both through the C ABI: outputs bit-identical
on two calls in a row, the second with a smaller input (fewer rows, a shorter cache, another
split count), so stale partials from the first call cannot leak into the second. Oversized calls
are rejected on the host before anything launches."""
import pytest
import torch

from attn_cases import BF, D

pytestmark = pytest.mark.gpu
DEV = "cuda"
INVALID = 1  # hipErrorInvalidValue


def _case(g, n, hq, hkv, L, pos):
    kc = torch.randn(hkv, L, D, device=DEV, generator=g).to(BF)
    vc = torch.randn(hkv, L, D, device=DEV, generator=g).to(BF)
    q = torch.randn(n, hq * D, device=DEV, generator=g).to(BF)
    qg = torch.randn(n, hq * 2 * D, device=DEV, generator=g).to(BF)
    return kc, vc, q, qg, torch.tensor([pos], dtype=torch.int32, device=DEV)


def test_noalloc_decode_matches_decode(capi):
    g = torch.Generator(device=DEV).manual_seed(11)
    # (rows, Hq, Hkv, cache length, pos of row 0, split count); the second call is smaller
    for n, hq, hkv, L, pos, ns in ((8, 24, 4, 4096 + 8, 4096, 64), (2, 24, 4, 1000, 990, 16)):
        kc, vc, q, qg, p = _case(g, n, hq, hkv, L, pos)
        ref = torch.empty(n, hq * D, dtype=BF, device=DEV)
        got = torch.full((n, hq * D), float("nan"), dtype=BF, device=DEV)
        po = torch.empty(n, hq, ns, D, device=DEV)
        pml = torch.empty(n, hq, ns, 2, device=DEV)
        assert capi.decode(q, kc, vc, p, qg, hq * 2 * D, po, pml, ref, hq * D, n, hq, hkv, L,
                           ns) == 0
        assert capi.decode_noalloc(q, kc, vc, p, qg, hq * 2 * D, got, hq * D, n, hq, hkv, L,
                                   ns) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got, ref), (n, L, ns)


def test_noalloc_rejects_oversized_calls(capi):
    """n * Hq * NS above the array's capacity, and the decode's own limits, fail on the host."""
    g = torch.Generator(device=DEV).manual_seed(12)
    kc, vc, q, qg, p = _case(g, 8, 24, 4, 256, 100)
    out = torch.empty(8, 24 * D, dtype=BF, device=DEV)
    cap = capi.NOALLOC_MAX_SLOTS
    ns_over = cap // (8 * 24) + 1
    assert capi.decode_noalloc(q, kc, vc, p, qg, 48 * D, out, 24 * D, 8, 24, 4, 256,
                               ns_over) == INVALID
    assert capi.decode_noalloc(q, kc, vc, p, qg, 48 * D, out, 24 * D, 9, 24, 4, 256,
                               4) == INVALID
    torch.cuda.synchronize()
