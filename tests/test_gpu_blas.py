"""GPU: the direct hipBLASLt GEMMs (testt_amd/blas.py, soupk_gemm_lt).  With the tuned table
accepted, the layer's GEMMs at 2048 tokens run the table's solution and give torch.matmul's
result bit for bit; other problems (the heuristic's choice) within the fp16 bound of float64
sums (1 ulp plus 64 * 2^-24 * sum|terms|); bias, accumulation, strided rows, the batched fp32
form, the fallbacks, and replays of a captured HIP graph."""

import pytest
import torch

from testt_amd import _ext, blas, gemm_tuning

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def within(got, exact, terms):
    h = exact.to(got.dtype)
    inf = torch.tensor(float("inf"), dtype=got.dtype, device=h.device)
    ulp = (torch.nextafter(h.abs(), inf) - h.abs()).double()
    err = (got.double() - exact).abs()
    bad = err > ulp + 64 * 2.0 ** -24 * terms
    assert not bool(bad.any()), f"{int(bad.sum())} of {bad.numel()} beyond, max {float(err.max()):.3g}"


def rnd(*shape, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).to(torch.float16).to(DEV)


@pytest.fixture(scope="module")
def tuned():
    accepted = gemm_tuning.enable()
    yield accepted
    gemm_tuning.disable()


# the layer's GEMMs at 2048 tokens: (kind, N, K); tn: x [M, K] @ W[N, K]^T, nn: dy [M, N] @ W
LAYER = [("tn", 2048, 1536, True), ("tn", 1536, 1536, False), ("tn", 17920, 1536, False),
         ("tn", 1536, 8960, False), ("nn", 2048, 1536, False), ("nn", 1536, 1536, False),
         ("nn", 1536, 8960, False), ("nn", 17920, 1536, False)]


@pytest.mark.parametrize("kind,N,K,with_bias", LAYER)
def test_layer_gemms_match_torch(tuned, kind, N, K, with_bias):
    if not tuned:
        pytest.skip("the tuned table's validators do not match this system")
    print(f"blas {kind} N={N} K={K} bias={with_bias}", flush=True)
    M = 2048
    W = rnd(N, K, scale=K ** -0.5, seed=N + K)
    b = rnd(N, scale=0.1, seed=3) if with_bias else None
    if kind == "tn":
        x = rnd(M, K, seed=1)
        got = blas.linear(x, W, b)
        ref = torch.nn.functional.linear(x, W, b)
        key = ("tn", N, M, K, K, K, N, with_bias)
        args = (1, 0, N, M, K, K, 0, K, 0, N, 0, 0, 1, int(with_bias), 0)
    else:
        dy = rnd(M, N, scale=0.1, seed=2)
        got = blas.matmul(dy, W)
        ref = torch.mm(dy, W)
        key = ("nn", K, M, N, K, N, K, False)
        args = (0, 0, K, M, N, K, 0, N, 0, K, 0, 0, 1, 0, 0)
    torch.cuda.synchronize()
    want = blas._table.get(key, -1)
    ran = _ext.lib().soupk_gemm_lt_index(*args, want, blas.WORKSPACE_BYTES)
    if want >= 0:
        assert ran == want                        # the table's solution ran
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,N,K", [(888, 2048, 1536), (77, 1536, 8960), (1, 256, 64),
                                   (300, 384, 128)])
def test_heuristic_problems_within_fp16_bound(M, N, K):
    print(f"blas heuristic M={M} N={N} K={K}", flush=True)
    x, W = rnd(M, K, seed=5), rnd(N, K, scale=K ** -0.5, seed=6)
    got = blas.linear(x, W)
    within(got, x.double() @ W.double().t(), x.double().abs() @ W.double().abs().t())
    dy = rnd(M, N, scale=0.1, seed=7)
    got = blas.matmul(dy, W)
    within(got, dy.double() @ W.double(), dy.double().abs() @ W.double().abs())


def test_bias_accumulate_and_strided_rows():
    M, N, K = 200, 384, 512
    x, W, b = rnd(M, K, seed=8), rnd(N, K, scale=K ** -0.5, seed=9), rnd(N, scale=0.1, seed=10)
    y = blas.linear(x, W, b)
    xd, Wd = x.double(), W.double()
    within(y, xd @ Wd.t() + b.double(), xd.abs() @ Wd.abs().t() + b.double().abs())
    # rows of a wider buffer: the same result
    wide = torch.zeros(M, K + 64, dtype=torch.float16, device=DEV)
    wide[:, :K] = x
    assert torch.equal(blas.linear(wide[:, :K], W, b), y)
    # out += dy @ W
    dy = rnd(M, N, scale=0.1, seed=11)
    acc = rnd(M, K, scale=0.1, seed=12)
    exact = acc.double() + dy.double() @ Wd
    blas.matmul(dy, W, out=acc, accumulate=True)
    within(acc, exact, exact.abs() + dy.double().abs() @ Wd.abs())


def test_batched_fp32():
    P, M, K, N = 4, 256, 640, 384
    a = rnd(M, P * K, seed=13)
    bmat = rnd(P * K, N, scale=0.05, seed=14)
    a3 = a.as_strided((P, M, K), (K, a.stride(0), 1))
    b3 = bmat.as_strided((P, K, N), (K * bmat.stride(0), bmat.stride(0), 1))
    got = blas.bmm_f32(a3, b3)
    assert got.dtype == torch.float32 and got.shape == (P, M, N)
    exact = torch.einsum("pmk,pkn->pmn", a3.double(), b3.double())
    terms = torch.einsum("pmk,pkn->pmn", a3.double().abs(), b3.double().abs())
    assert bool(((got.double() - exact).abs() <= 64 * 2.0 ** -24 * terms + 1e-30).all())


def test_fallbacks_give_torch_results():
    M, N, K = 64, 128, 96
    x, W = rnd(M, K, seed=15), rnd(N, K, seed=16)
    # fp32 operands, a misaligned view: torch's own path
    assert torch.equal(blas.linear(x.float(), W.float()), torch.mm(x.float(), W.float().t()))
    buf = torch.zeros(M * K + 1, dtype=torch.float16, device=DEV)
    xm = buf[1:].view(M, K)
    xm.copy_(x)
    assert torch.equal(blas.linear(xm, W), torch.mm(xm, W.t()))
    with pytest.raises(ValueError):
        blas.matmul(x, W.t(), accumulate=True)


def test_invalid_arguments_rejected(tuned):
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_lt", 2, 0, 8, 8, 8, 16, 8, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1,
                  None, 0, None)                   # trans flag 2
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_lt", 0, 0, 8, 8, 8, 16, 4, 0, 16, 8, 0, 16, 8, 0, 0, 1, 0, None, -1,
                  None, 0, None)                   # lda < m


def test_graph_replays_match_eager():
    """A captured blas.matmul replayed three times, eager work in between, equals the eager
    result each time."""
    M, N, K = 512, 1536, 1536
    x, W = rnd(M, K, seed=17), rnd(N, K, scale=K ** -0.5, seed=18)
    eager = blas.linear(x, W)
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        blas.matmul(x, W.t(), out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        blas.matmul(x, W.t(), out=out)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        blas.linear(rnd(M, K, seed=19 + i), W)       # eager work between replays
        torch.cuda.synchronize()
