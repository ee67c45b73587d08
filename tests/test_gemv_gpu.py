"""GPU parity tests of gemv_bf16 (the projections on either side of the attention path) against
the CPU oracle, with the reference's own bars (tests/test_kernels.py:75-115 of qengine):
  * |y - y_exact| <= 2^-8 |y_exact| + K 2^-23 sum|w x| with y_exact in fp64, every element;
  * vs the reference kernel's own fp32 summation order (oracle.gemv_bf16_ref): within one bf16
    ulp for > 99% of the elements (the reference test asks the same of cuBLAS);
  * row r of an nr-row call is bit-identical to a 1-row call, also for strided rows;
  * NaN in x reaches every output.
"""
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _rand(g, *shape):
    return torch.randn(*shape, generator=g).to(BF)


def _check(out: torch.Tensor, W: torch.Tensor, x: torch.Tensor):
    err = (out.double() - O.gemv_exact(W, x)).abs()
    bound = O.gemv_bound(W, x)
    assert bool((err <= bound).all()), (err / bound).max().item()
    ref = O.gemv_bf16_ref(W, x).float()
    near = (out.float() - ref).abs() <= 2.0 ** -7 * out.float().abs() + 1e-6
    assert near.float().mean().item() > 0.99


@pytest.mark.parametrize("N,K", [(1, 8), (7, 64), (127, 1000), (1000, 1024), (4097, 1024),
                                 (6144, 1024), (1024, 3584), (5120, 17408), (248320, 1024),
                                 (33, 24)])
def test_gemv_bf16(native, N, K):
    g = torch.Generator().manual_seed(N * 7 + K)
    W, x = _rand(g, N, K), _rand(g, K)
    out = torch.empty(N, dtype=BF, device=DEV)
    native.gemv_bf16(W.to(DEV), x.to(DEV), out)
    _check(out.cpu().view(1, N), W, x)


@pytest.mark.parametrize("nr", [1, 5, 8])
@pytest.mark.parametrize("N,K", [(14336, 5120), (5120, 6144)])
def test_attention_projection_shapes(native, nr, N, K):
    """The attention branch's in_proj ([q|gate] x 24 + k + v = 14,336 rows of 5,120) and o_proj
    (5,120 rows of 6,144) at 1, 5 (MTP verify) and 8 rows."""
    g = torch.Generator().manual_seed(N + nr)
    W, x = (torch.randn(N, K, generator=g) * K ** -0.5).to(BF), _rand(g, nr, K)
    out = torch.empty(nr, N, dtype=BF, device=DEV)
    native.gemv_bf16(W.to(DEV), x.to(DEV), out)
    _check(out.cpu(), W, x)


@pytest.mark.parametrize("nr", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("N,K", [(7, 64), (1000, 1024), (6144, 1024), (1024, 3584), (33, 24),
                                 (5120, 6144)])
def test_gemv_rows_bit_exact(native, nr, N, K):
    """Row r of an nr-row call == a 1-row call on that row, bit for bit, with row strides larger
    than the widths (views into wider buffers)."""
    g = torch.Generator(device=DEV).manual_seed(nr * 1000 + N)
    W = torch.randn(N, K, device=DEV, generator=g).to(BF)
    xb = torch.randn(nr, K + 16, device=DEV, generator=g).to(BF)
    x = xb[:, :K]
    ob = torch.empty(nr, N + 8, dtype=BF, device=DEV)
    out = ob[:, :N]
    native.gemv_bf16(W, x, out)
    one = torch.empty(N, dtype=BF, device=DEV)
    for r in range(nr):
        native.gemv_bf16(W, x[r].contiguous(), one)
        assert torch.equal(out[r], one), r


@pytest.mark.parametrize("nr", [1, 2, 5, 8])
def test_gemv_tile_height_keeps_bits(native, capi, nr):
    """Row prefixes of one weight cut into tiles of 10, 16, 14 and 12 rows (qe_gemv_tile_rows on
    256 CUs) give the same bits for every shared row: an output does not depend on its row's
    place in a tile. Both kernels (1-2 rows LDS-staged, 3-8 rows register activations)."""
    K = 2048
    g = torch.Generator(device=DEV).manual_seed(31 + nr)
    W = torch.randn(5120, K, device=DEV, generator=g).to(BF)
    x = torch.randn(nr, K, device=DEV, generator=g).to(BF)
    full = torch.empty(nr, 5120, dtype=BF, device=DEV)
    native.gemv_bf16(W, x, full)
    heights = {}
    for N in (5120, 4096, 3584, 3072, 2560, 1000):
        heights[N] = capi.gemv_tile_rows(N, K)
        assert capi.gemv_kparts(N, K) == 4
        out = torch.empty(nr, N, dtype=BF, device=DEV)
        native.gemv_bf16(W[:N], x, out)
        assert torch.equal(out, full[:, :N]), (N, heights[N])
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert heights == {5120: 10, 4096: 16, 3584: 14, 3072: 12, 2560: 10, 1000: 10}
    _check(full.cpu(), W.cpu(), x.cpu())


@pytest.mark.parametrize("nr", [1, 3, 6, 8])
@pytest.mark.parametrize("N,K", [(100, 8), (300, 264), (64, 520), (2000, 4104)])
def test_gemv_partial_k_blocks(native, nr, N, K):
    """K not a multiple of the 256-k block (and K < 256): the chunks past K in the last block
    must contribute nothing, whatever the neighbouring row holds (here NaN past each x row)."""
    g = torch.Generator().manual_seed(N + K + nr)
    W, xw = _rand(g, N, K), _rand(g, nr, K + 8)
    xw[:, K:] = float("nan")
    x = xw[:, :K]
    out = torch.empty(nr, N, dtype=BF, device=DEV)
    native.gemv_bf16(W.to(DEV), xw.to(DEV)[:, :K], out)
    _check(out.cpu(), W, x)


def test_gemv_graph_replays(native):
    """Captured in a hipGraph and replayed with new activations between replays: every replay
    matches an eager call."""
    W = torch.randn(3000, 2048, device=DEV).to(BF)
    x = torch.randn(2, 2048, device=DEV).to(BF)
    out = torch.empty(2, 3000, dtype=BF, device=DEV)
    ref = torch.empty_like(out)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.gemv_bf16(W, x, out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.gemv_bf16(W, x, out)
    for rep in range(4):
        x.copy_(torch.randn(2, 2048, device=DEV).to(BF))
        g.replay()
        native.gemv_bf16(W, x, ref)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), rep


def test_gemv_leaves_the_output_padding_alone(native):
    W = torch.randn(100, 64, device=DEV).to(BF)
    x = torch.randn(3, 64, device=DEV).to(BF)
    ob = torch.full((3, 108), 7.0, dtype=BF, device=DEV)
    native.gemv_bf16(W, x, ob[:, :100])
    assert bool((ob[:, 100:] == 7.0).all())


def test_gemv_nan_propagates(native):
    W = torch.randn(64, 128, device=DEV).to(BF)
    x = torch.randn(128, device=DEV).to(BF)
    x[3] = float("nan")
    out = torch.empty(64, dtype=BF, device=DEV)
    native.gemv_bf16(W, x, out)
    assert torch.isnan(out).all()


def test_capi_gemv_matches_extension(native, capi):
    """The C ABI (ctypes) gives the extension's bits."""
    g = torch.Generator(device=DEV).manual_seed(9)
    W = torch.randn(777, 1000, device=DEV, generator=g).to(BF)
    x = torch.randn(4, 1000, device=DEV, generator=g).to(BF)
    a = torch.empty(4, 777, dtype=BF, device=DEV)
    b = torch.empty_like(a)
    native.gemv_bf16(W, x, a)
    assert capi.gemv_bf16(W, x, b, 4, 777, 1000, 1000, 777) == 0
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_hbm_read_probe_runs(capi):
    buf = torch.ones(1 << 22, dtype=torch.int32, device=DEV)
    sink = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert capi.hbm_read_probe(buf, buf.numel() * 4, sink) == 0
    torch.cuda.synchronize()
    assert sink.item() == 0
