"""qe_attn_decode_noalloc (the decode with the library's own device scratch) against
qe_attn_decode with caller-owned part_o / part_ml, both through the C ABI: outputs bit-identical
on two calls in a row, the second with a smaller input (fewer rows, a shorter cache, another
split count), so stale partials from the first call cannot leak into the second; and under
hipGraph capture, replayed with changed inputs. Oversized calls are rejected on the host before
anything launches."""
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


def test_noalloc_decode_under_graph_capture(capi):
    """qe_attn_decode_noalloc captured into a hipGraph (torch.cuda.graph, the capture stream as
    the call's stream) after one eager call on the device: replays after the inputs change in
    place (new q, gate, cache rows and position) equal eager qe_attn_decode with caller scratch,
    bit for bit, with eager noalloc calls of another shape between the replays."""
    g = torch.Generator(device=DEV).manual_seed(13)
    n, hq, hkv, L, ns = 2, 24, 4, 2048, 48
    kc, vc, q, qg, p = _case(g, n, hq, hkv, L, 1500)
    out = torch.empty(n, hq * D, dtype=BF, device=DEV)
    assert capi.decode_noalloc(q, kc, vc, p, qg, hq * 2 * D, out, hq * D, n, hq, hkv, L, ns) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert capi.decode_noalloc(q, kc, vc, p, qg, hq * 2 * D, out, hq * D, n, hq, hkv, L,
                                   ns) == 0
    po = torch.empty(n, hq, ns, D, device=DEV)
    pml = torch.empty(n, hq, ns, 2, device=DEV)
    ref = torch.empty_like(out)
    other = _case(g, 1, 8, 2, 700, 650)
    other_out = torch.empty(1, 8 * D, dtype=BF, device=DEV)
    for r, pos in enumerate((1500, 1900, 900, 2047)):
        q.copy_(torch.randn(q.shape, device=DEV, generator=g).to(BF))
        qg.copy_(torch.randn(qg.shape, device=DEV, generator=g).to(BF))
        kc[:, pos - 8: pos + 1] = torch.randn(hkv, 9, D, device=DEV, generator=g).to(BF)
        p.fill_(pos)
        out.fill_(float("nan"))
        graph.replay()
        assert capi.decode(q, kc, vc, p, qg, hq * 2 * D, po, pml, ref, hq * D, n, hq, hkv, L,
                           ns) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(out, ref), r
        kc2, vc2, q2, qg2, p2 = other  # an eager call of another shape shares the array
        assert capi.decode_noalloc(q2, kc2, vc2, p2, qg2, 16 * D, other_out, 8 * D, 1, 8, 2, 700,
                                   16) == 0
        torch.cuda.synchronize()


def test_noalloc_rejects_oversized_calls(capi):
    """n * Hq * NS above the array's capacity, and the decode's own limits, fail on the host."""
    g = torch.Generator(device=DEV).manual_seed(12)
    kc, vc, q, qg, p = _case(g, 8, 24, 4, 256, 100)
    out = torch.empty(8, 24 * D, dtype=BF, device=DEV)
    cap = capi.NOALLOC_MAX_SLOTS
    ns_over = cap // (8 * 24) + 1
    assert capi.decode_noalloc(q, kc, vc, p, qg, 48 * D, out, 24 * D, 8, 24, 4, 256,
                               ns_over) == INVALID
    assert capi.decode_noalloc(q, kc, vc, p, qg, 48 * D, out, 24 * D, 65536, 24, 4, 256,
                               4) == INVALID
    assert capi.decode_noalloc(q, kc, vc, p, qg, 48 * D, out, 24 * D, 8, 25, 4, 256,
                               4) == INVALID
    torch.cuda.synchronize()
